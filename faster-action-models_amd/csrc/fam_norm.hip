// Row-normalisation kernels: AdaLN-Zero / LayerNorm and RMSNorm + rotary embedding.
//
// One 64-lane wavefront owns one row; a 256-thread workgroup handles four rows.  Each
// lane reads 16-byte vectors (8 x bf16) at column (v*64 + lane)*8, so a wavefront's
// load instruction covers 1 KB of contiguous row.  Rows up to 4096 wide stay in
// registers between the statistics and the output pass (NV = 8-element vectors per
// lane); wider rows are re-read (the second read hits L2).
//
// Bytes per row (the roofline numerator):  AdaLN  2*D (x) + 2*D (y) + modulation;
// RMSNorm+RoPE  2*D + 2*D + tables.  Both are HBM-bound streaming kernels.
#include "fam_common.h"

namespace fam {

struct AdalnArgs {
  const bf16* x; int64_t xrs;
  const bf16* shift; const bf16* scale; int64_t mbs, mrs;
  const bf16* w; const bf16* b;
  bf16* y; int64_t yrs;
  int64_t rows, rpb, dim;
  float eps;
};

// AFF: the LayerNorm affine is present.  MOD: no AdaLN shift-scale (0), one per row (1, an
// HBM stream: loaded with x), or one per batch (2, an L2-resident row, loaded after the
// statistics).  Both modulated forms hold NV shift and NV scale vectors next to x (about 96
// registers at NV = 8), so they run at the same occupancy; compile-time, because occupancy is
// what keeps HBM busy here.
template <int NV, bool AFF, int MOD>
__global__ __launch_bounds__(256) void adaln_kernel(AdalnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r0 >= a.rows) return;  // wave-uniform
  const int64_t D = a.dim;
  const float invD = 1.0f / (float)D;

  // LayerNorm of 8 elements (two-pass statistics given), then affine and modulation
  auto finish = [&](const float* xv, float mean, float rstd, bf16x8 wv, bf16x8 bv, bf16x8 sh, bf16x8 sc) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (xv[e] - mean) * rstd;
    if (AFF && a.w) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= to_f(wv[e]);
    }
    if (AFF && a.b) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += to_f(bv[e]);
    }
    if (MOD) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = o[e] * (1.0f + to_f(sc[e])) + to_f(sh[e]);
    }
    bf16x8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = to_bf(o[e]);
    return out;
  };

  if constexpr (NV > 0) {
    // Every load of the row (x, LayerNorm affine, per-row shift / scale) is issued before the
    // statistics, so a wave waits for memory once; x stays bf16 in registers and is widened in
    // each pass.
    constexpr int NA = AFF ? NV : 1, NMD = MOD != 0 ? NV : 1;
    bf16x8 xv8[1][NV], wv[NA], bv[NA], sh[NMD], sc[NMD];
    constexpr int RPW = 1;
    auto col = [&](int i) { const int64_t c = ((int64_t)i * 64 + lane) * 8; return c < D ? c : 0; };
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int64_t r = r0 + k < a.rows ? r0 + k : a.rows - 1;
#pragma unroll
      for (int i = 0; i < NV; ++i) xv8[k][i] = load8(a.x + r * a.xrs + col(i));
    }
    if constexpr (AFF) {
      // an absent weight or bias reads x instead (a valid address; finish ignores the value):
      // a load under a branch, or a select on its value, would wait for the x loads before it
      const bf16* wsrc = a.w ? a.w : a.x;
      const bf16* bsrc = a.b ? a.b : a.x;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        wv[i] = load8(wsrc + col(i));
        bv[i] = load8(bsrc + col(i));
      }
    }
    if constexpr (MOD == 1) {
      const int64_t bidx = r0 / a.rpb, sidx = r0 - bidx * a.rpb;
      const int64_t moff = bidx * a.mbs + sidx * a.mrs;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        sh[i] = load8(a.shift + moff + col(i));
        sc[i] = load8(a.scale + moff + col(i));
      }
    }
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int64_t r = r0 + k;
      if (r >= a.rows) break;   // wave-uniform
      const int64_t bidx = r / a.rpb, sidx = r - bidx * a.rpb;
      const int64_t moff = bidx * a.mbs + sidx * a.mrs;
      bf16* yr = a.y + r * a.yrs;
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (((int64_t)i * 64 + lane) * 8 < D) {
#pragma unroll
          for (int e = 0; e < 8; ++e) s += to_f(xv8[k][i][e]);
        }
      }
      const float mean = wave_sum_valu(s) * invD;
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (((int64_t)i * 64 + lane) * 8 < D) {
#pragma unroll
          for (int e = 0; e < 8; ++e) { const float d = to_f(xv8[k][i][e]) - mean; q += d * d; }
        }
      }
      const float rstd = rsqrtf(wave_sum_valu(q) * invD + a.eps);
      if constexpr (MOD == 2) {
        // the batch's shift / scale row (L2-resident), all of it in one round trip
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          sh[i] = load8(a.shift + moff + col(i));
          sc[i] = load8(a.scale + moff + col(i));
        }
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int64_t c = ((int64_t)i * 64 + lane) * 8;
        if (c < D) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = to_f(xv8[k][i][e]);
          store8(yr + c, finish(v, mean, rstd, wv[AFF ? i : 0], bv[AFF ? i : 0], sh[MOD != 0 ? i : 0],
                                sc[MOD != 0 ? i : 0]));
        }
      }
    }
  } else {
    // wide rows: three passes over x (the re-reads hit L2)
    const int64_t r = r0;
    const bf16* xr = a.x + r * a.xrs;
    const int64_t bidx = r / a.rpb, sidx = r - bidx * a.rpb;
    const int64_t moff = bidx * a.mbs + sidx * a.mrs;
    bf16* yr = a.y + r * a.yrs;
    float s = 0.f;
    for (int64_t c = (int64_t)lane * 8; c < D; c += 512) {
      bf16x8 t = load8(xr + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += to_f(t[e]);
    }
    const float mean = wave_sum_valu(s) * invD;
    float q = 0.f;
    for (int64_t c = (int64_t)lane * 8; c < D; c += 512) {
      bf16x8 t = load8(xr + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float d = to_f(t[e]) - mean; q += d * d; }
    }
    const float rstd = rsqrtf(wave_sum_valu(q) * invD + a.eps);
    for (int64_t c = (int64_t)lane * 8; c < D; c += 512) {
      bf16x8 t = load8(xr + c);
      float xv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] = to_f(t[e]);
      const bf16x8 z = t;
      store8(yr + c, finish(xv, mean, rstd, AFF && a.w ? load8(a.w + c) : z, AFF && a.b ? load8(a.b + c) : z,
                            MOD ? load8(a.shift + moff + c) : z, MOD ? load8(a.scale + moff + c) : z));
    }
  }
}

struct RmsRopeArgs {
  const bf16* x; int64_t xrs;
  bf16* y; int64_t yrs;
  int64_t rows, seq, dim;
  const bf16* w; float eps;
  const float* cs; const float* sn; int64_t trs, tes, hd;
  int64_t wgp;   // weight groups: row r is scaled by w + (r % wgp) * dim
};

template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(RmsRopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.rows) return;  // wave-uniform
  const bf16* xr = a.x + r * a.xrs;
  const int64_t D = a.dim;

  // All loads of the row happen before any store, so y == x (in place) is safe: each
  // lane rewrites exactly the 8 elements it read.
  bf16x8 in[NV > 0 ? NV : 1];
  float q = 0.f;
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = ((int64_t)i * 64 + lane) * 8;
      in[i] = (c < D) ? load8(xr + c) : zero8();
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float f = to_f(in[i][e]); q += f * f; }
    }
  } else {
    for (int64_t c = (int64_t)lane * 8; c < D; c += 512) {
      bf16x8 t = load8(xr + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float f = to_f(t[e]); q += f * f; }
    }
  }
  const float rs = a.w ? rsqrtf(wave_sum_valu(q) / (float)D + a.eps) : 1.0f;
  const int64_t pos = r % a.seq;
  bf16* yr = a.y + r * a.yrs;
  const bf16* wr = a.w ? a.w + (r % a.wgp) * D : nullptr;
  auto emit = [&](int64_t c, bf16x8 t) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_f(t[e]);
    if (a.w) {
      // RMSNorm rounds to the storage dtype before the weight multiply (FB/wan_video_dit.py:166-167).
      bf16x8 wv = load8(wr + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_f(to_bf(to_f(to_bf(o[e] * rs)) * to_f(wv[e])));
    }
    if (a.cs) {
      const int64_t j0 = (c % a.hd) >> 1;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int64_t t = pos * a.trs + (j0 + p) * a.tes;
        const float cc = a.cs[t], ss = a.sn[t];
        const float x0 = o[2 * p], x1 = o[2 * p + 1];
        o[2 * p] = x0 * cc - x1 * ss;
        o[2 * p + 1] = x0 * ss + x1 * cc;
      }
    }
    bf16x8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = to_bf(o[e]);
    store8(yr + c, out);
  };
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = ((int64_t)i * 64 + lane) * 8;
      if (c < D) emit(c, in[i]);
    }
  } else {
    // Wide rows: not in registers; out-of-place only (checked on the host).
    for (int64_t c = (int64_t)lane * 8; c < D; c += 512) emit(c, load8(xr + c));
  }
}

// Row-in-registers form of rmsnorm_rope_kernel for dim <= 64 * 8 * NV with the rotation
// tables read as 16-byte vectors (TAB 0: no rotation; 1: separate cos / sin rows, element
// stride 1; 2: interleaved (cos, sin) pairs).  Every load of the row -- x, the weight and the
// table entries -- is issued before the sum of squares, so a wave waits for memory once.
// TSH: hd divides 512, so the pairs of lane's chunk (i * 64 + lane) * 8 do not depend on i and
// the table entries are read once per lane and row.  RPW: rows per wave (a wave owns rows
// RPW * w .. RPW * w + RPW - 1 and issues the loads of all of them at once, sharing the weight).
template <int NV, int TAB, bool TSH, int RPW>
__global__ __launch_bounds__(256) void rmsnorm_rope_vec_kernel(RmsRopeArgs a) {
  constexpr int NT = TSH ? 1 : NV;   // table vectors per row
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (r0 >= a.rows) return;  // wave-uniform
  const int D = (int)a.dim, hd = (int)a.hd;
  // without a weight the weight loads read x (a valid address, value unused): an unconditional
  // load joins the others in one wait, where a load under a branch waits for those before it
  const bf16* wr = a.w ? a.w + (r0 % a.wgp) * (int64_t)D : a.x;   // RPW > 1 only with one group
  bf16x8 in[RPW][NV], wv[NV];
  f32x4 t0[RPW][NT], t1[RPW][NT];
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int64_t r = r0 + k < a.rows ? r0 + k : a.rows - 1;
    const bf16* xr = a.x + r * a.xrs;
    const int pos = (int)(r % a.seq);
    const float* crow = a.cs + (int64_t)pos * a.trs;
    const float* srow = a.sn + (int64_t)pos * a.trs;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8, cc = c < D ? c : 0;
      in[k][i] = load8(xr + cc);
      if (k == 0) wv[i] = load8(wr + cc);
      if (i < NT) {
        const int j0 = ((TSH ? lane * 8 : cc) % hd) >> 1;   // first of the 4 rotation pairs of these 8 elements
        if constexpr (TAB == 1) {
          t0[k][i] = *reinterpret_cast<const f32x4*>(crow + j0);
          t1[k][i] = *reinterpret_cast<const f32x4*>(srow + j0);
        } else if constexpr (TAB == 2) {
          t0[k][i] = *reinterpret_cast<const f32x4*>(crow + 2 * j0);       // c0 s0 c1 s1
          t1[k][i] = *reinterpret_cast<const f32x4*>(crow + 2 * j0 + 4);   // c2 s2 c3 s3
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    if (r0 + k >= a.rows) break;  // wave-uniform
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const bool ok = (i * 64 + lane) * 8 < D;
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float f = ok ? to_f(in[k][i][e]) : 0.f; q += f * f; }
    }
    const float rs = a.w ? rsqrtf(wave_sum_valu(q) / (float)D + a.eps) : 1.0f;
    bf16* yr = a.y + (r0 + k) * a.yrs;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * 64 + lane) * 8;
      if (c >= D) continue;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = to_f(in[k][i][e]);
      if (a.w) {
        // RMSNorm rounds to the storage dtype before the weight multiply (FB/wan_video_dit.py:166-167).
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_f(to_bf(to_f(to_bf(o[e] * rs)) * to_f(wv[i][e])));
      }
      if constexpr (TAB != 0) {
        const int ti = TSH ? 0 : i;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          float cc, ss;
          if constexpr (TAB == 1) {
            cc = t0[k][ti][p];
            ss = t1[k][ti][p];
          } else {
            cc = p < 2 ? t0[k][ti][2 * p] : t1[k][ti][2 * p - 4];
            ss = p < 2 ? t0[k][ti][2 * p + 1] : t1[k][ti][2 * p - 3];
          }
          const float x0 = o[2 * p], x1 = o[2 * p + 1];
          o[2 * p] = x0 * cc - x1 * ss;
          o[2 * p + 1] = x0 * ss + x1 * cc;
        }
      }
      bf16x8 out;
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = to_bf(o[e]);
      store8(yr + c, out);
    }
  }
}

}  // namespace fam

using namespace fam;

template <int NV, int MOD>
static void launch_adaln_m(const AdalnArgs& a, bool aff, hipStream_t s) {
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  if (aff) FAM_LAUNCH((adaln_kernel<NV, true, MOD>), grid, dim3(256), 0, s, a);
  else FAM_LAUNCH((adaln_kernel<NV, false, MOD>), grid, dim3(256), 0, s, a);
}
// mod: 0 none, 1 per row, 2 per batch (mod_row_stride 0)
template <int NV>
static void launch_adaln(const AdalnArgs& a, bool aff, int mod, hipStream_t s) {
  if (mod == 1) launch_adaln_m<NV, 1>(a, aff, s);
  else if (mod == 2) launch_adaln_m<NV, 2>(a, aff, s);
  else launch_adaln_m<NV, 0>(a, aff, s);
}

static int nv_for(int64_t dim) {
  const int64_t nv = (dim + 511) / 512;
  if (nv <= 1) return 1;
  if (nv <= 2) return 2;
  if (nv <= 4) return 4;
  if (nv <= 6) return 6;
  if (nv <= 8) return 8;
  return 0;
}

extern "C" int fam_adaln(const void* x, int64_t x_row_stride, const void* shift, const void* scale,
                         int64_t mod_batch_stride, int64_t mod_row_stride, const void* ln_weight,
                         const void* ln_bias, void* y, int64_t y_row_stride, int64_t rows,
                         int64_t rows_per_batch, int64_t dim, float eps, void* stream) {
  FAM_REQUIRE(x && y, FAM_ERR_INVALID_ARG, "fam_adaln: x and y must be non-null");
  FAM_REQUIRE(rows >= 0 && dim >= 8 && dim <= 16384 && dim % 8 == 0, FAM_ERR_INVALID_ARG,
              "fam_adaln: need dim %% 8 == 0 and 8 <= dim <= 16384 (dim=%lld)", (long long)dim);
  FAM_REQUIRE((shift == nullptr) == (scale == nullptr), FAM_ERR_INVALID_ARG,
              "fam_adaln: shift and scale must both be given or both be null");
  FAM_REQUIRE(rows_per_batch >= 1, FAM_ERR_INVALID_ARG, "fam_adaln: rows_per_batch must be >= 1");
  FAM_REQUIRE(x_row_stride >= dim && y_row_stride >= dim && x_row_stride % 8 == 0 && y_row_stride % 8 == 0,
              FAM_ERR_INVALID_ARG, "fam_adaln: row strides must be >= dim and multiples of 8");
  FAM_REQUIRE(fam_host::aligned16(x) && fam_host::aligned16(y), FAM_ERR_INVALID_ARG,
              "fam_adaln: x and y must be 16-byte aligned");
  FAM_REQUIRE(!shift || (fam_host::aligned16(shift) && fam_host::aligned16(scale) &&
                         mod_batch_stride % 8 == 0 && mod_row_stride % 8 == 0),
              FAM_ERR_INVALID_ARG, "fam_adaln: shift/scale must be 16-byte aligned with strides %% 8 == 0");
  FAM_REQUIRE((!ln_weight || fam_host::aligned16(ln_weight)) && (!ln_bias || fam_host::aligned16(ln_bias)),
              FAM_ERR_INVALID_ARG, "fam_adaln: ln_weight/ln_bias must be 16-byte aligned");
  if (rows == 0) return FAM_OK;
  AdalnArgs a{(const bf16*)x, x_row_stride, (const bf16*)shift, (const bf16*)scale, mod_batch_stride,
              mod_row_stride, (const bf16*)ln_weight, (const bf16*)ln_bias, (bf16*)y, y_row_stride,
              rows, rows_per_batch, dim, eps};
  hipStream_t s = (hipStream_t)stream;
  const bool aff = ln_weight || ln_bias;
  const int mod = shift == nullptr ? 0 : (mod_row_stride == 0 && rows_per_batch > 1 ? 2 : 1);
  switch (nv_for(dim)) {
    case 1: launch_adaln<1>(a, aff, mod, s); break;
    case 2: launch_adaln<2>(a, aff, mod, s); break;
    case 4: launch_adaln<4>(a, aff, mod, s); break;
    case 6: launch_adaln<6>(a, aff, mod, s); break;
    case 8: launch_adaln<8>(a, aff, mod, s); break;
    default: launch_adaln<0>(a, aff, mod, s); break;
  }
  return fam_host::check_launch("fam_adaln");
}

static int rmsnorm_rope_impl(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows,
                             int64_t seq_len, int64_t dim, const void* weight, int64_t groups, float eps,
                             const float* cos_tab, const float* sin_tab, int64_t tab_row_stride,
                             int64_t tab_elem_stride, int64_t head_dim, void* stream) {
  FAM_REQUIRE(x && y, FAM_ERR_INVALID_ARG, "fam_rmsnorm_rope: x and y must be non-null");
  FAM_REQUIRE(rows >= 0 && dim >= 8 && dim <= 16384 && dim % 8 == 0, FAM_ERR_INVALID_ARG,
              "fam_rmsnorm_rope: need dim %% 8 == 0 and 8 <= dim <= 16384 (dim=%lld)", (long long)dim);
  FAM_REQUIRE(x_row_stride >= dim && y_row_stride >= dim && x_row_stride % 8 == 0 && y_row_stride % 8 == 0,
              FAM_ERR_INVALID_ARG, "fam_rmsnorm_rope: row strides must be >= dim and multiples of 8");
  FAM_REQUIRE(fam_host::aligned16(x) && fam_host::aligned16(y) && (!weight || fam_host::aligned16(weight)),
              FAM_ERR_INVALID_ARG, "fam_rmsnorm_rope: x, y, weight must be 16-byte aligned");
  FAM_REQUIRE((cos_tab == nullptr) == (sin_tab == nullptr), FAM_ERR_INVALID_ARG,
              "fam_rmsnorm_rope: cos_tab and sin_tab must both be given or both be null");
  if (cos_tab) {
    FAM_REQUIRE(head_dim >= 8 && head_dim % 8 == 0 && dim % head_dim == 0, FAM_ERR_INVALID_ARG,
                "fam_rmsnorm_rope: head_dim must be a multiple of 8 dividing dim (head_dim=%lld)",
                (long long)head_dim);
    FAM_REQUIRE(seq_len >= 1, FAM_ERR_INVALID_ARG, "fam_rmsnorm_rope: seq_len must be >= 1");
  }
  const int nv = nv_for(dim);
  FAM_REQUIRE(nv != 0 || x != y, FAM_ERR_UNSUPPORTED, "fam_rmsnorm_rope: in-place needs dim <= 4096");
  if (rows == 0) return FAM_OK;
  RmsRopeArgs a{(const bf16*)x, x_row_stride, (bf16*)y, y_row_stride, rows, seq_len > 0 ? seq_len : 1, dim,
                (const bf16*)weight, eps, cos_tab, sin_tab, tab_row_stride, tab_elem_stride,
                head_dim > 0 ? head_dim : 8, groups};
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  // vector table reads: rows of 16-byte aligned fp32 with 4 consecutive pairs per 8 elements
  const auto al16 = [](const void* p) { return fam_host::aligned16(p); };
  int tab = 3;
  if (!cos_tab) tab = 0;
  else if (tab_elem_stride == 1 && tab_row_stride % 4 == 0 && al16(cos_tab) && al16(sin_tab)) tab = 1;
  else if (tab_elem_stride == 2 && sin_tab == cos_tab + 1 && tab_row_stride % 4 == 0 && al16(cos_tab)) tab = 2;
  if (nv != 0 && tab != 3 && dim <= (int64_t)1 << 30) {
    const bool tsh = 512 % a.hd == 0;
    // two rows per wave once there are enough rows to fill the machine with half the waves
    const bool two = rows >= 4096 && nv <= 6 && groups == 1;
    const dim3 grid2((unsigned)((rows + 7) / 8));
#define FAM_RR_VEC2(NV, TAB, TSH)                                                                          \
  do {                                                                                                     \
    if (two) FAM_LAUNCH((rmsnorm_rope_vec_kernel<NV, TAB, TSH, 2>), grid2, block, 0, s, a);                \
    else FAM_LAUNCH((rmsnorm_rope_vec_kernel<NV, TAB, TSH, 1>), grid, block, 0, s, a);                     \
  } while (0)
#define FAM_RR_VEC(NV)                                      \
  switch (tab) {                                            \
    case 0: FAM_RR_VEC2(NV, 0, false); break;               \
    case 1:                                                 \
      if (tsh) FAM_RR_VEC2(NV, 1, true);                    \
      else FAM_RR_VEC2(NV, 1, false);                       \
      break;                                                \
    default:                                                \
      if (tsh) FAM_RR_VEC2(NV, 2, true);                    \
      else FAM_RR_VEC2(NV, 2, false);                       \
      break;                                                \
  }
    switch (nv) {
      case 1: FAM_RR_VEC(1); break;
      case 2: FAM_RR_VEC(2); break;
      case 4: FAM_RR_VEC(4); break;
      case 6: FAM_RR_VEC(6); break;
      default: FAM_RR_VEC(8); break;
    }
#undef FAM_RR_VEC
#undef FAM_RR_VEC2
    return fam_host::check_launch("fam_rmsnorm_rope");
  }
  switch (nv) {
    case 1: FAM_LAUNCH(rmsnorm_rope_kernel<1>, grid, block, 0, s, a); break;
    case 2: FAM_LAUNCH(rmsnorm_rope_kernel<2>, grid, block, 0, s, a); break;
    case 4: FAM_LAUNCH(rmsnorm_rope_kernel<4>, grid, block, 0, s, a); break;
    case 6: FAM_LAUNCH(rmsnorm_rope_kernel<6>, grid, block, 0, s, a); break;
    case 8: FAM_LAUNCH(rmsnorm_rope_kernel<8>, grid, block, 0, s, a); break;
    default: FAM_LAUNCH(rmsnorm_rope_kernel<0>, grid, block, 0, s, a); break;
  }
  return fam_host::check_launch("fam_rmsnorm_rope");
}

extern "C" int fam_rmsnorm_rope(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride,
                                int64_t rows, int64_t seq_len, int64_t dim, const void* weight, float eps,
                                const float* cos_tab, const float* sin_tab, int64_t tab_row_stride,
                                int64_t tab_elem_stride, int64_t head_dim, void* stream) {
  return rmsnorm_rope_impl(x, x_row_stride, y, y_row_stride, rows, seq_len, dim, weight, 1, eps, cos_tab, sin_tab,
                           tab_row_stride, tab_elem_stride, head_dim, stream);
}

extern "C" int fam_rmsnorm_grouped(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride,
                                   int64_t rows, int64_t dim, const void* weights, int64_t groups, float eps,
                                   void* stream) {
  FAM_REQUIRE(weights && groups >= 1, FAM_ERR_INVALID_ARG, "fam_rmsnorm_grouped: need weights and groups >= 1");
  FAM_REQUIRE(rows % groups == 0, FAM_ERR_INVALID_ARG, "fam_rmsnorm_grouped: rows must be a multiple of groups");
  return rmsnorm_rope_impl(x, x_row_stride, y, y_row_stride, rows, 1, dim, weights, groups, eps, nullptr, nullptr,
                           0, 0, 0, stream);
}

// ---------------------------------------------------------------------------------------
// Per-head RMSNorm + rotate-half RoPE (the Cosmos backbone's q / k: RMSNorm(head_dim) with a
// head_dim-wide weight shared by the heads, then apply_rotary_emb(use_real=True,
// use_real_unbind_dim=-2), whose pairs are (d, d + head_dim / 2)).
//
// One thread owns 8 consecutive elements (16 bytes) of one head; the LPH = head_dim / 8 lanes of
// a head are consecutive lanes of one wave (a segment's width is a whole number of heads, so a
// head never straddles a wave), its sum of squares is an xor-shuffle reduction over them, and
// the rotation partner of element d -- d + head_dim / 2 or d - head_dim / 2 -- sits in lane
// l ^ (LPH / 2) at the same position.  Loads (x, weight, the table rows) are issued first.
// Bytes per row segment: 2 * width (x) + 2 * width (y); the weight and the tables are L2-resident.
namespace fam {
struct HeadNormArgs {
  const bf16* x; int64_t xrs;
  bf16* y; int64_t yrs;
  int64_t rows, seq, nseg, seg_stride, width;
  const bf16* w; int64_t wss;
  float eps;
  const float* cs; const float* sn; int64_t trs;
  uint32_t total;   // rows * nseg * width / 8 threads
};

template <int LPH, bool ROPE>
__global__ __launch_bounds__(256) void headnorm_rope_kernel(HeadNormArgs a) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= a.total) return;   // a head's lanes share the test: total is a multiple of LPH
  const uint32_t cpr = (uint32_t)(a.width >> 3), cps = cpr * (uint32_t)a.nseg;
  const uint32_t r = t / cps, rem = t - r * cps;
  const uint32_t seg = rem / cpr, c = rem - seg * cpr;
  const uint32_t cl = c & (LPH - 1);                      // chunk within the head
  const int64_t col = (int64_t)seg * a.seg_stride + (int64_t)c * 8;
  const bf16x8 v = load8(a.x + (int64_t)r * a.xrs + col);
  const bf16x8 w = load8(a.w + (int64_t)seg * a.wss + cl * 8);
  f32x4 c0, c1, s0, s1;
  if constexpr (ROPE) {
    const int64_t pos = (int64_t)(r % (uint32_t)a.seq);
    const float* cp = a.cs + pos * a.trs + cl * 8;
    const float* sp = a.sn + pos * a.trs + cl * 8;
    c0 = *reinterpret_cast<const f32x4*>(cp);
    c1 = *reinterpret_cast<const f32x4*>(cp + 4);
    s0 = *reinterpret_cast<const f32x4*>(sp);
    s1 = *reinterpret_cast<const f32x4*>(sp + 4);
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += to_f(v[e]) * to_f(v[e]);
#pragma unroll
  for (int o = LPH / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, kWave);
  const float rstd = rsqrtf(ss * (1.0f / (float)(LPH * 8)) + a.eps);
  float n[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = to_f(to_bf(to_f(to_bf(to_f(v[e]) * rstd)) * to_f(w[e])));
  bf16x8 o;
  if constexpr (ROPE) {
    // rotated = cat(-x[D/2:], x[:D/2]): the first half takes minus its partner, the second plus
    const float sg = cl < (uint32_t)(LPH / 2) ? -1.f : 1.f;
    const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __shfl_xor(n[e], LPH / 2, kWave);
      o[e] = to_bf(n[e] * cv[e] + sg * p * sv[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf(n[e]);
  }
  store8(a.y + (int64_t)r * a.yrs + col, o);
}
}  // namespace fam

extern "C" int fam_headnorm_rope(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows,
                                 int64_t seq_len, int64_t nseg, int64_t seg_stride, int64_t width, int64_t head_dim,
                                 const void* weight, int64_t weight_seg_stride, float eps, const float* cos_tab,
                                 const float* sin_tab, int64_t tab_row_stride, void* stream) {
  using namespace fam;
  FAM_REQUIRE(x && y && weight, FAM_ERR_INVALID_ARG, "fam_headnorm_rope: x, y and weight must be non-null");
  FAM_REQUIRE(head_dim >= 16 && head_dim <= 512 && (head_dim & (head_dim - 1)) == 0, FAM_ERR_INVALID_ARG,
              "fam_headnorm_rope: head_dim must be a power of two in [16, 512] (got %lld)", (long long)head_dim);
  FAM_REQUIRE(rows >= 0 && nseg >= 1 && width >= head_dim && width % head_dim == 0, FAM_ERR_INVALID_ARG,
              "fam_headnorm_rope: need rows >= 0, nseg >= 1 and width a multiple of head_dim");
  FAM_REQUIRE(seg_stride % 8 == 0 && x_row_stride % 8 == 0 && y_row_stride % 8 == 0 && weight_seg_stride % 8 == 0 &&
                  (nseg == 1 || seg_stride >= width) &&
                  x_row_stride >= (nseg - 1) * seg_stride + width && y_row_stride >= (nseg - 1) * seg_stride + width,
              FAM_ERR_INVALID_ARG,
              "fam_headnorm_rope: strides must be multiples of 8 elements and the segments must fit the rows");
  FAM_REQUIRE(fam_host::aligned16(x) && fam_host::aligned16(y) && fam_host::aligned16(weight), FAM_ERR_INVALID_ARG,
              "fam_headnorm_rope: x, y and weight must be 16-byte aligned");
  FAM_REQUIRE((cos_tab == nullptr) == (sin_tab == nullptr), FAM_ERR_INVALID_ARG,
              "fam_headnorm_rope: cos_tab and sin_tab must both be given or both be null");
  if (cos_tab)
    FAM_REQUIRE(seq_len >= 1 && tab_row_stride >= head_dim && tab_row_stride % 4 == 0 &&
                    fam_host::aligned16(cos_tab) && fam_host::aligned16(sin_tab),
                FAM_ERR_INVALID_ARG,
                "fam_headnorm_rope: tables need seq_len >= 1, a row stride >= head_dim (multiple of 4) and "
                "16-byte alignment");
  const int64_t total = rows * nseg * (width / 8);
  FAM_REQUIRE(total < ((int64_t)1 << 32) - 256, FAM_ERR_UNSUPPORTED, "fam_headnorm_rope: too many elements");
  if (total == 0) return FAM_OK;
  HeadNormArgs a{(const bf16*)x, x_row_stride, (bf16*)y, y_row_stride, rows, seq_len > 0 ? seq_len : 1, nseg,
                 seg_stride, width, (const bf16*)weight, weight_seg_stride, eps, cos_tab, sin_tab, tab_row_stride,
                 (uint32_t)total};
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
#define FAM_HN(L)                                                                         \
  do {                                                                                    \
    if (cos_tab) FAM_LAUNCH((headnorm_rope_kernel<L, true>), grid, block, 0, s, a);       \
    else FAM_LAUNCH((headnorm_rope_kernel<L, false>), grid, block, 0, s, a);              \
  } while (0)
  switch (head_dim) {
    case 16: FAM_HN(2); break;
    case 32: FAM_HN(4); break;
    case 64: FAM_HN(8); break;
    case 128: FAM_HN(16); break;
    case 256: FAM_HN(32); break;
    default: FAM_HN(64); break;
  }
#undef FAM_HN
  return fam_host::check_launch("fam_headnorm_rope");
}
