// Row kernel of the fused action expert: one workgroup per output row.
//
//   v[n] = source(m, n) + bias[n]            source: the split-K partials of fam_gemm_partial
//                                            summed in split order, or a small-K linear
//   v    = act(v)                            (GELU-tanh / SiLU)
//   v    = res[m, n] + gate(m, n) * v        (optional residual update)
//   out[m, n] = v                            (bf16, or fp32 for the fp32 latents)
//   then, on the stored row, the normalisation the NEXT operation needs:
//     LayerNorm (optional affine) or AdaLN modulate over the whole row, or RMSNorm (+ RoPE)
//     over up to two column segments (the q and k parts of a fused QKV row)  -> nout
//
// Because a workgroup holds the whole row, the row statistics need no second kernel and no
// cross-workgroup traffic; the block reductions run through LDS in a fixed order.
// Bytes per row: 4*splits*N (partials) + 2*N (out) [+ 2*N residual] [+ 2*N nout].
#include "fam_common.h"

namespace fam {

struct RowArgs {
  int src;
  const float* part; int64_t splits, split_stride;
  const float* xin; int64_t ldx, kin; const bf16* win;
  int64_t M, N;
  const bf16* bias; int act;
  const void* res; int64_t ldr;
  const bf16* gate; int64_t gbs, grs, gns; int64_t rpb;
  void* out; int64_t ldo; int out_f32;
  int norm; float eps;
  const bf16* nw; const bf16* nb;
  const bf16* shift; const bf16* scale; int64_t mbs, mrs;
  int nseg; int64_t seg0[2]; int64_t segw; const bf16* segwt[2];
  const float* cs; const float* sn; int64_t trs, tes, hd, seq;
  bf16* nout; int64_t ldn;
  int64_t ldp;   // row stride of the partial planes
};

constexpr int RT = 256;  // threads per row

__device__ __forceinline__ float act_fn(float v, int act) {
  if (act == FAM_ACT_GELU_TANH) return gelu_tanh(v);
  if (act == FAM_ACT_SILU) return silu(v);
  if (act == FAM_ACT_RELU) return fmaxf(v, 0.f);
  if (act == FAM_ACT_GELU_ERF) return gelu_erf(v);
  return v;
}

// Sum over the 256 threads of the workgroup; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // red may still be read by a previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// NV groups of 4 columns per thread: N <= 4 * RT * NV.
template <int NV>
__global__ __launch_bounds__(RT) void rowop_kernel(RowArgs a) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t m = blockIdx.x;
  const int64_t bi = m / a.rpb, si = m - bi * a.rpb;
  float v[NV][4];
  bool ok[NV][4];

#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = ((int64_t)tid + RT * j) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[j][e] = 0.f; ok[j][e] = c + e < a.N; }
    if (a.src == 0) {
      if ((a.N & 3) == 0) {
        if (c < a.N) {
          const float* p = a.part + m * a.ldp + c;
#pragma unroll 8
          for (int64_t z = 0; z < a.splits; ++z) {
            const f32x4 t = *reinterpret_cast<const f32x4*>(p + z * a.split_stride);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j][e] += t[e];
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (ok[j][e])
            for (int64_t z = 0; z < a.splits; ++z) v[j][e] += a.part[z * a.split_stride + m * a.ldp + c + e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (ok[j][e])
          for (int64_t k = 0; k < a.kin; ++k) v[j][e] += a.xin[m * a.ldx + k] * to_f(a.win[(c + e) * a.kin + k]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (!ok[j][e]) continue;
      const int64_t n = c + e;
      float x = v[j][e];
      if (a.bias) x += to_f(a.bias[n]);
      x = act_fn(x, a.act);
      if (a.res) {
        float g = 1.0f;
        if (a.gate) g = to_f(a.gate[bi * a.gbs + si * a.grs + n * a.gns]);
        const float r = a.out_f32 ? reinterpret_cast<const float*>(a.res)[m * a.ldr + n]
                                  : to_f(reinterpret_cast<const bf16*>(a.res)[m * a.ldr + n]);
        x = r + g * x;
      }
      if (a.out_f32) {
        reinterpret_cast<float*>(a.out)[m * a.ldo + n] = x;
      } else {
        const bf16 xb = to_bf(x);
        reinterpret_cast<bf16*>(a.out)[m * a.ldo + n] = xb;
        x = to_f(xb);  // the stored (rounded) value feeds the normalisation
      }
      v[j][e] = x;
    }
  }
  if (a.norm == FAM_ROWNORM_NONE) return;

  if (a.norm == FAM_ROWNORM_LAYERNORM || a.norm == FAM_ROWNORM_ADALN) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += ok[j][e] ? v[j][e] : 0.f;
    const float mean = block_sum(s, red) / (float)a.N;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = ok[j][e] ? v[j][e] - mean : 0.f;
        q += d * d;
      }
    const float rstd = rsqrtf(block_sum(q, red) / (float)a.N + a.eps);
    const int64_t moff = bi * a.mbs + si * a.mrs;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!ok[j][e]) continue;
        const int64_t n = ((int64_t)tid + RT * j) * 4 + e;
        float o = (v[j][e] - mean) * rstd;
        if (a.norm == FAM_ROWNORM_LAYERNORM) {
          if (a.nw) o *= to_f(a.nw[n]);
          if (a.nb) o += to_f(a.nb[n]);
        } else {
          o = o * (1.0f + to_f(a.scale[moff + n])) + to_f(a.shift[moff + n]);
        }
        a.nout[m * a.ldn + n] = to_bf(o);
      }
    return;
  }

  // RMSNorm (+ RoPE) over column segments [seg0[g], seg0[g] + segw)
  const int64_t pos = m % a.seq;
  for (int sg = 0; sg < a.nseg; ++sg) {
    const int64_t c0 = a.seg0[sg];
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t n = ((int64_t)tid + RT * j) * 4 + e;
        if (ok[j][e] && n >= c0 && n < c0 + a.segw) q += v[j][e] * v[j][e];
      }
    const float rs = rsqrtf(block_sum(q, red) / (float)a.segw + a.eps);
    const bf16* wt = a.segwt[sg];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t cb = ((int64_t)tid + RT * j) * 4;
      if (cb < c0 || cb >= c0 + a.segw || cb >= a.N) continue;  // segments are 4-aligned
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)  // bf16 before the weight multiply, as RMSNorm.forward
        o[e] = to_f(to_bf(to_f(to_bf(v[j][e] * rs)) * to_f(wt[cb - c0 + e])));
      if (a.cs) {
        const int64_t j0 = ((cb - c0) % a.hd) >> 1;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int64_t t = pos * a.trs + (j0 + p) * a.tes;
          const float cc = a.cs[t], ss = a.sn[t];
          const float x0 = o[2 * p], x1 = o[2 * p + 1];
          o[2 * p] = x0 * cc - x1 * ss;
          o[2 * p + 1] = x0 * ss + x1 * cc;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) a.nout[m * a.ldn + cb + e] = to_bf(o[e]);
    }
  }
}


// ---------------------------------------------------------------------------------------
// rowop_vec_kernel: the split-K source with every operand 4-column aligned.  NW waves hold
// 4 consecutive columns per thread (N <= 256 * NW); all global loads of the row (up to
// MAXS partial planes, bias, residual, gate, modulation, norm weights, RoPE tables) are
// issued before the first use, so a row costs one memory round trip instead of one per
// operand (one more per further MAXS planes of a long-K split plan).
__device__ __forceinline__ void ld4(const bf16* p, float o[4]) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = to_f(v[e]);
}

template <int NW>
__device__ __forceinline__ float block_sum_nw(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += red[w];
  return t;
}

template <int NW>
__device__ __forceinline__ void block_sum2_nw(float& a, float& b, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  a = wave_sum(a);
  b = wave_sum(b);
  __syncthreads();
  if (lane == 0) { red[wave] = a; red[NW + wave] = b; }
  __syncthreads();
  float ta = 0.f, tb = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) { ta += red[w]; tb += red[NW + w]; }
  a = ta;
  b = tb;
}

template <int NW, int MAXS>
__global__ __launch_bounds__(NW * 64) void rowop_vec_kernel(RowArgs a) {
  __shared__ float red[2 * NW];
  const int tid = threadIdx.x;
  // 32-bit index arithmetic (M, rows_per_batch, seq_len and head_dim are < 2^31, checked on
  // the host): a 64-bit division is a ~100-instruction sequence on the critical path
  const uint32_t m32 = blockIdx.x, rpb32 = (uint32_t)a.rpb;
  const int64_t m = m32;
  const int64_t bi = m32 / rpb32, si = m32 - (uint32_t)bi * rpb32;
  // rows wider than one workgroup (no normalisation only) are tiled over grid.y
  const int64_t c = (int64_t)blockIdx.y * (NW * 256) + (int64_t)tid * 4;
  const bool act = c < a.N;
  const int64_t cs = act ? c : 0;  // a valid column for inactive threads' loads

  // ---- phase 1: every load of the row, raw, from always-valid addresses (an absent operand
  // reads the partials instead), so that no wait can be scheduled between the loads
  const float* safe = a.part;
  f32x4 pz[MAXS];
  const int64_t ns = a.splits;
#pragma unroll
  for (int z = 0; z < MAXS; ++z) {
    const int64_t zz = z < ns ? z : ns - 1;
    pz[z] = *reinterpret_cast<const f32x4*>(a.part + zz * a.split_stride + m * a.ldp + cs);
  }
  auto raw4 = [&](const bf16* p) { return *reinterpret_cast<const uint2*>(p ? (const void*)p : (const void*)safe); };
  const uint2 r_bias = raw4(a.bias ? a.bias + cs : nullptr);
  const bool res_f32 = a.res && a.out_f32, res_bf = a.res && !a.out_f32;
  const f32x4 r_resf = *reinterpret_cast<const f32x4*>(res_f32 ? reinterpret_cast<const float*>(a.res) + m * a.ldr + cs : safe);
  const uint2 r_resb = raw4(res_bf ? reinterpret_cast<const bf16*>(a.res) + m * a.ldr + cs : nullptr);
  const bf16* gp = a.gate ? a.gate + bi * a.gbs + si * a.grs : nullptr;
  const uint2 r_gate4 = raw4(gp && a.gns ? gp + cs : nullptr);
  const bf16 r_gate1 = *(gp && !a.gns ? gp : reinterpret_cast<const bf16*>(safe));
  // norm operands: (scale, shift) for AdaLN, (weight, bias) for LayerNorm, weight for RMS
  const int64_t mo = bi * a.mbs + si * a.mrs;
  const bf16* p_na = nullptr;
  const bf16* p_nb = nullptr;
  int seg = -1;
  const bf16* sw0 = a.segwt[0];
  const bf16* sw1 = a.segwt[1];
  const int64_t s0 = a.seg0[0], s1 = a.seg0[1], sgw = a.segw;
  int64_t cl = 0;
  if (a.norm == FAM_ROWNORM_ADALN) {
    p_na = a.scale + mo + cs;
    p_nb = a.shift + mo + cs;
  } else if (a.norm == FAM_ROWNORM_LAYERNORM) {
    p_na = a.nw ? a.nw + cs : nullptr;
    p_nb = a.nb ? a.nb + cs : nullptr;
  } else if (a.norm == FAM_ROWNORM_RMS) {
    if (a.nseg > 0 && c >= s0 && c < s0 + sgw) seg = 0;
    if (a.nseg > 1 && c >= s1 && c < s1 + sgw) seg = 1;
    if (!act) seg = -1;
    cl = c - (seg == 1 ? s1 : s0);
    p_na = seg == 0 ? sw0 + cl : (seg == 1 ? sw1 + cl : nullptr);
  }
  const uint2 r_na = raw4(p_na), r_nb = raw4(p_nb);
  // RoPE table entries of the thread's two pairs
  const bool rope = a.cs != nullptr && seg >= 0;
  int64_t t0 = 0, t1 = 0;
  if (rope) {
    const int64_t pos = m32 % (uint32_t)a.seq, j0 = ((uint32_t)cl % (uint32_t)a.hd) >> 1;
    t0 = pos * a.trs + j0 * a.tes;
    t1 = t0 + a.tes;
  }
  const float* tc = rope ? a.cs : safe;
  const float* tsn = rope ? a.sn : safe;
  const float rc0 = tc[t0], rc1 = tc[t1], rs0 = tsn[t0], rs1 = tsn[t1];
  __builtin_amdgcn_sched_barrier(0);

  // ---- unpack
  auto unpack = [](uint2 r, float o[4]) {
    bf16x4 v;
    __builtin_memcpy(&v, &r, 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = to_f(v[e]);
  };
  float bias[4] = {0.f, 0.f, 0.f, 0.f}, res[4] = {0.f, 0.f, 0.f, 0.f}, gate[4] = {1.f, 1.f, 1.f, 1.f};
  if (a.bias) unpack(r_bias, bias);
  if (res_f32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) res[e] = r_resf[e];
  } else if (res_bf) {
    unpack(r_resb, res);
  }
  if (gp) {
    if (a.gns) {
      unpack(r_gate4, gate);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) gate[e] = to_f(r_gate1);
    }
  }
  float na[4] = {1.f, 1.f, 1.f, 1.f}, nb[4] = {0.f, 0.f, 0.f, 0.f};
  if (p_na) unpack(r_na, na);
  if (p_nb) unpack(r_nb, nb);
  const float rc[2] = {rope ? rc0 : 1.f, rope ? rc1 : 1.f}, rsn[2] = {rope ? rs0 : 0.f, rope ? rs1 : 0.f};

  // ---- phase 2: sum the planes in split order, epilogue, store
  float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int z = 0; z < MAXS; ++z)
    if (z < ns) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += pz[z][e];
    }
  // planes past the first MAXS (long-K split plans): further batches of MAXS loads, still in
  // split order
  for (int64_t z0 = MAXS; z0 < ns; z0 += MAXS) {
#pragma unroll
    for (int z = 0; z < MAXS; ++z) {
      const int64_t zz = z0 + z < ns ? z0 + z : ns - 1;
      pz[z] = *reinterpret_cast<const f32x4*>(a.part + zz * a.split_stride + m * a.ldp + cs);
    }
#pragma unroll
    for (int z = 0; z < MAXS; ++z)
      if (z0 + z < ns) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += pz[z][e];
      }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float x = act_fn(v[e] + bias[e], a.act);
    if (a.res) x = res[e] + gate[e] * x;
    v[e] = x;
  }
  if (a.out_f32) {
    if (act) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[e];
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + m * a.ldo + c) = o;
    }
  } else {
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = to_bf(v[e]);
      v[e] = to_f(o[e]);  // the stored (rounded) value feeds the normalisation
    }
    if (act) *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16*>(a.out) + m * a.ldo + c) = o;
  }
  if (a.norm == FAM_ROWNORM_NONE) return;

  bf16x4 o;
  if (a.norm == FAM_ROWNORM_LAYERNORM || a.norm == FAM_ROWNORM_ADALN) {
    const float s = act ? (v[0] + v[1]) + (v[2] + v[3]) : 0.f;
    const float mean = block_sum_nw<NW>(s, red) / (float)a.N;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = act ? v[e] - mean : 0.f;
      q += d * d;
    }
    const float rstd = rsqrtf(block_sum_nw<NW>(q, red) / (float)a.N + a.eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y = (v[e] - mean) * rstd;
      o[e] = to_bf(a.norm == FAM_ROWNORM_LAYERNORM ? y * na[e] + nb[e] : y * (1.0f + na[e]) + nb[e]);
    }
    if (act) *reinterpret_cast<bf16x4*>(a.nout + m * a.ldn + c) = o;
    return;
  }

  // RMSNorm over each segment (one combined reduction for both), then RoPE on the pairs
  float q0 = 0.f, q1 = 0.f;
  if (act && seg >= 0) {
    const float q = (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
    if (seg == 0) q0 = q; else q1 = q;
  }
  block_sum2_nw<NW>(q0, q1, red);
  if (!act || seg < 0) return;
  const float rs = rsqrtf((seg == 0 ? q0 : q1) / (float)a.segw + a.eps);
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)  // bf16 before the weight multiply, as RMSNorm.forward
    y[e] = to_f(to_bf(to_f(to_bf(v[e] * rs)) * na[e]));
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float x0 = y[2 * p], x1 = y[2 * p + 1];
    y[2 * p] = x0 * rc[p] - x1 * rsn[p];
    y[2 * p + 1] = x0 * rsn[p] + x1 * rc[p];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = to_bf(y[e]);
  *reinterpret_cast<bf16x4*>(a.nout + m * a.ldn + c) = o;
}

}  // namespace fam

using namespace fam;

// The vectorised kernel takes the split-K source with <= 16 planes when every operand row
// starts on a 4-column boundary; anything else runs the generic per-element kernel.
static bool vec_eligible(const fam_rowop_desc* d) {
  auto al = [](const void* p, unsigned b) { return (reinterpret_cast<uintptr_t>(p) & (b - 1)) == 0; };
  if (d->src != FAM_ROWSRC_PARTIALS || d->N % 4 != 0 || d->splits > 64 || d->ldo % 4 != 0) return false;
  if (d->ldp % 4 != 0) return false;
  if (!al(d->out, d->out_f32 ? 16 : 8) || (d->bias && !al(d->bias, 8))) return false;
  if (d->res && (d->ldr % 4 != 0 || !al(d->res, d->out_f32 ? 16 : 8))) return false;
  if (d->gate && !(d->gate_ns == 0 || (d->gate_ns == 1 && d->gate_bs % 4 == 0 && d->gate_rs % 4 == 0 &&
                                       al(d->gate, 8))))
    return false;
  if (d->norm != FAM_ROWNORM_NONE && (d->ldn % 4 != 0 || !al(d->nout, 8))) return false;
  if (d->norm == FAM_ROWNORM_ADALN &&
      (d->mod_bs % 4 != 0 || d->mod_rs % 4 != 0 || !al(d->shift, 8) || !al(d->scale, 8)))
    return false;
  if (d->norm == FAM_ROWNORM_LAYERNORM && ((d->ln_weight && !al(d->ln_weight, 8)) || (d->ln_bias && !al(d->ln_bias, 8))))
    return false;
  if (d->norm == FAM_ROWNORM_RMS)
    for (int g = 0; g < d->nseg; ++g)
      if (!al(d->seg_weight[g], 8)) return false;
  return true;
}

// Rows wider than one workgroup are tiled over grid.y, one tile of 256 NW columns per
// workgroup: without normalisation any tiling works; an RMS row tiles when every segment is
// exactly one tile (the q | k | v row of a fused projection, each segment normalised inside
// its own workgroup).  Returns the waves per workgroup, or 0 when the row does not tile.
static int rms_tile_waves(const fam_rowop_desc* d) {
  if (d->norm != FAM_ROWNORM_RMS || d->seg_width % 256 != 0) return 0;
  const int64_t nw = d->seg_width / 256;
  if (nw != 4 && nw != 8 && nw != 12 && nw != 16) return 0;
  for (int g = 0; g < d->nseg && g < 2; ++g)
    if (d->seg_col0[g] % d->seg_width != 0) return 0;
  return (int)nw;
}

extern "C" int fam_rowop(const fam_rowop_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_rowop: null descriptor");
  FAM_REQUIRE(d->M >= 0 && d->N >= 1 &&
                  (d->N <= 4 * RT * 4 ||
                   (d->N < (1LL << 30) && (d->norm == FAM_ROWNORM_NONE || rms_tile_waves(d) > 0) && vec_eligible(d))),
              FAM_ERR_INVALID_ARG,
              "fam_rowop: need 1 <= N <= 4096, or a wider row on the vectorised path (N %% 4 == 0, partials "
              "source, aligned operands) without normalisation or with RMS segments of one tile each (N=%lld)",
              (long long)d->N);
  FAM_REQUIRE(d->out, FAM_ERR_INVALID_ARG, "fam_rowop: out must be non-null");
  FAM_REQUIRE(d->ldo >= d->N, FAM_ERR_INVALID_ARG, "fam_rowop: ldo must be >= N");
  if (d->src == FAM_ROWSRC_PARTIALS) {
    const int64_t ldp = d->ldp > 0 ? d->ldp : d->N;
    FAM_REQUIRE(ldp >= d->N && (d->M == 0 || d->split_stride >= (d->M - 1) * ldp + d->N), FAM_ERR_INVALID_ARG,
                "fam_rowop: need ldp >= N and split_stride >= (M - 1) * ldp + N");
    FAM_REQUIRE(d->partials && d->splits >= 1 && d->split_stride >= d->M * d->N, FAM_ERR_INVALID_ARG,
                "fam_rowop: partials need splits >= 1 and split_stride >= M*N");
    FAM_REQUIRE(d->N % 4 != 0 || fam_host::aligned16(d->partials), FAM_ERR_INVALID_ARG,
                "fam_rowop: partials must be 16-byte aligned");
    FAM_REQUIRE(d->N % 4 != 0 || d->split_stride % 4 == 0, FAM_ERR_INVALID_ARG,
                "fam_rowop: split_stride must be a multiple of 4");
  } else if (d->src == FAM_ROWSRC_SMALLK) {
    FAM_REQUIRE(d->x_in && d->w_in && d->k_in >= 1 && d->k_in <= 64 && d->ldx >= d->k_in, FAM_ERR_INVALID_ARG,
                "fam_rowop: small-K source needs x_in, w_in and 1 <= k_in <= 64");
  } else {
    FAM_REQUIRE(false, FAM_ERR_INVALID_ARG, "fam_rowop: unknown source %d", d->src);
  }
  FAM_REQUIRE(d->act >= FAM_ACT_NONE && d->act <= FAM_ACT_GELU_ERF, FAM_ERR_INVALID_ARG, "fam_rowop: unknown act");
  FAM_REQUIRE(!d->gate || d->res, FAM_ERR_INVALID_ARG, "fam_rowop: a gate needs a residual");
  FAM_REQUIRE(d->rows_per_batch >= 1, FAM_ERR_INVALID_ARG, "fam_rowop: rows_per_batch must be >= 1");
  FAM_REQUIRE(d->norm >= FAM_ROWNORM_NONE && d->norm <= FAM_ROWNORM_RMS, FAM_ERR_INVALID_ARG, "fam_rowop: unknown norm");
  if (d->norm != FAM_ROWNORM_NONE) {
    FAM_REQUIRE(!d->out_f32, FAM_ERR_UNSUPPORTED, "fam_rowop: normalisation needs a bf16 row");
    FAM_REQUIRE(d->nout && d->ldn >= d->N, FAM_ERR_INVALID_ARG, "fam_rowop: norm output missing or ldn < N");
  }
  if (d->norm == FAM_ROWNORM_ADALN) {
    FAM_REQUIRE(d->shift && d->scale, FAM_ERR_INVALID_ARG, "fam_rowop: AdaLN needs shift and scale");
  }
  if (d->norm == FAM_ROWNORM_RMS) {
    FAM_REQUIRE(d->nseg >= 1 && d->nseg <= 2 && d->seg_width >= 4 && d->seg_width % 4 == 0, FAM_ERR_INVALID_ARG,
                "fam_rowop: RMS needs 1 or 2 segments of a width that is a multiple of 4");
    for (int g = 0; g < d->nseg; ++g) {
      FAM_REQUIRE(d->seg_weight[g] && d->seg_col0[g] >= 0 && d->seg_col0[g] % 4 == 0 &&
                      d->seg_col0[g] + d->seg_width <= d->N,
                  FAM_ERR_INVALID_ARG, "fam_rowop: bad RMS segment %d", g);
    }
    FAM_REQUIRE((d->rope_cos == nullptr) == (d->rope_sin == nullptr), FAM_ERR_INVALID_ARG,
                "fam_rowop: rope_cos and rope_sin must both be given or both be null");
    if (d->rope_cos) {
      FAM_REQUIRE(d->head_dim >= 4 && d->head_dim % 4 == 0 && d->seg_width % d->head_dim == 0 && d->seq_len >= 1,
                  FAM_ERR_INVALID_ARG, "fam_rowop: RoPE needs head_dim %% 4 == 0 dividing the segment, seq_len >= 1");
    }
  }
  FAM_REQUIRE(d->M < (1LL << 31) && d->rows_per_batch < (1LL << 31) && d->seq_len < (1LL << 31) &&
                  d->head_dim < (1LL << 31),
              FAM_ERR_UNSUPPORTED, "fam_rowop: M, rows_per_batch, seq_len and head_dim must be < 2^31");
  if (d->M == 0) return FAM_OK;

  RowArgs a{};
  a.src = d->src;
  a.part = d->partials; a.splits = d->splits; a.split_stride = d->split_stride;
  a.ldp = d->ldp > 0 ? d->ldp : d->N;
  a.xin = d->x_in; a.ldx = d->ldx; a.kin = d->k_in; a.win = (const bf16*)d->w_in;
  a.M = d->M; a.N = d->N;
  a.bias = (const bf16*)d->bias; a.act = d->act;
  a.res = d->res; a.ldr = d->ldr;
  a.gate = (const bf16*)d->gate; a.gbs = d->gate_bs; a.grs = d->gate_rs; a.gns = d->gate_ns;
  a.rpb = d->rows_per_batch;
  a.out = d->out; a.ldo = d->ldo; a.out_f32 = d->out_f32 != 0;
  a.norm = d->norm; a.eps = d->eps;
  a.nw = (const bf16*)d->ln_weight; a.nb = (const bf16*)d->ln_bias;
  a.shift = (const bf16*)d->shift; a.scale = (const bf16*)d->scale; a.mbs = d->mod_bs; a.mrs = d->mod_rs;
  a.nseg = d->nseg; a.seg0[0] = d->seg_col0[0]; a.seg0[1] = d->seg_col0[1]; a.segw = d->seg_width;
  a.segwt[0] = (const bf16*)d->seg_weight[0]; a.segwt[1] = (const bf16*)d->seg_weight[1];
  a.cs = d->rope_cos; a.sn = d->rope_sin; a.trs = d->rope_row_stride; a.tes = d->rope_elem_stride;
  a.hd = d->head_dim > 0 ? d->head_dim : 4; a.seq = d->seq_len > 0 ? d->seq_len : 1;
  a.nout = (bf16*)d->nout; a.ldn = d->ldn;
  hipStream_t s = (hipStream_t)stream;
  if (vec_eligible(d)) {
    const int tw = d->N > 4096 ? rms_tile_waves(d) : 0;
    int nw = tw > 0 ? tw : (d->N <= 1024 ? 4 : (d->N <= 2048 ? 8 : (d->N <= 3072 ? 12 : 16)));
    // a wider row without normalisation tiles over grid.y: take the widest tile that divides it
    // (14336 = 7 x 2048), so that no workgroup of the last tile idles on missing columns
    if (tw == 0 && d->N > 4096 && d->N % (16 * 256) != 0)
      for (int w : {12, 8})
        if (d->N % (w * 256) == 0) {
          nw = w;
          break;
        }
    const dim3 grid((unsigned)d->M, (unsigned)((d->N + nw * 256 - 1) / (nw * 256)));
    const int ms = d->splits <= 4 ? 4 : (d->splits <= 8 ? 8 : 16);
#define FAM_ROWVEC(NW_, MS_) \
  if (nw == NW_ && ms == MS_) FAM_LAUNCH((rowop_vec_kernel<NW_, MS_>), grid, dim3(NW_ * 64), 0, s, a)
    FAM_ROWVEC(4, 4); FAM_ROWVEC(4, 8); FAM_ROWVEC(4, 16);
    FAM_ROWVEC(8, 4); FAM_ROWVEC(8, 8); FAM_ROWVEC(8, 16);
    FAM_ROWVEC(12, 4); FAM_ROWVEC(12, 8); FAM_ROWVEC(12, 16);
    FAM_ROWVEC(16, 4); FAM_ROWVEC(16, 8); FAM_ROWVEC(16, 16);
#undef FAM_ROWVEC
    return fam_host::check_launch("fam_rowop");
  }
  const dim3 grid((unsigned)d->M);
  if (d->N <= 4 * RT) FAM_LAUNCH(rowop_kernel<1>, grid, dim3(RT), 0, s, a);
  else if (d->N <= 8 * RT) FAM_LAUNCH(rowop_kernel<2>, grid, dim3(RT), 0, s, a);
  else FAM_LAUNCH(rowop_kernel<4>, grid, dim3(RT), 0, s, a);
  return fam_host::check_launch("fam_rowop");
}
