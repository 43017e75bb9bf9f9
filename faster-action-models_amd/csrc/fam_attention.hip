// Flash-style attention on bf16 MFMA (gfx950):  o = softmax(q k^T * scale + mask) v.
//
// Formulation.  Scores are computed transposed, S^T = K Q^T, with the key tile as the
// MFMA A-operand and the query tile as the B-operand (v_mfma_f32_16x16x32_bf16).  A lane
// then owns ONE query (column l%16) and four keys per 16-key sub-tile, so the running
// max / sum of the online softmax are per-lane scalars reduced over the 4 lane groups with
// two shuffles, and the probabilities already sit in the B-operand layout of the second
// product O^T = V^T P^T (A-operand = V^T read from a transposed LDS tile).  The key order
// inside an MFMA k-block is permuted consistently on both operands (keys {4g..4g+3} and
// {16+4g..16+4g+3} for lane group g), which leaves the dot products unchanged.
//
// Work split.  A workgroup of NW waves owns 16*NW queries of one (batch, head); K/V blocks
// of 32 keys are staged through LDS and shared by the waves.  For short query blocks
// (Sq <= 64, e.g. 32 action tokens over 1560 context tokens) the keys are additionally
// split over grid.z workgroups; each writes its unnormalised partial (O, m, l) and the last
// to arrive combines them in split order (deterministic, no float atomics).
//
// Algorithmic bytes per launch: 2*B*H*Dh*(2*Sq + 2*Sk) (+ mask); flops 4*B*H*Sq*Sk*Dh.
#include <algorithm>

#include "fam_common.h"

namespace fam {

constexpr int KB = 32;  // keys per LDS block

struct AttnArgs {
  const bf16* q; int64_t q_bs, q_rs, q_hs;
  const bf16* k0; int64_t k0_bs, k0_rs, k0_hs;
  const bf16* v0; int64_t v0_bs, v0_rs, v0_hs;
  const bf16* k1; int64_t k1_bs, k1_rs, k1_hs;
  const bf16* v1; int64_t v1_bs, v1_rs, v1_hs;
  bf16* o; int64_t o_bs, o_rs, o_hs;
  int64_t H, Sq, sk0, Sk, kchunk;
  float scale_log2;
  const void* mask; int mask_kind; int64_t mbs, mhs, mqs;
  int splits;
  unsigned* cnt; float* opart; float* mlpart;
  int64_t sq_pad;
};

template <int DH, int NW>
__global__ __launch_bounds__(NW * 64) void attn_kernel(AttnArgs a) {
  constexpr int NC = (DH + 31) / 32;   // 32-wide k-chunks of the head dim (zero padded)
  constexpr int NDT = (DH + 15) / 16;  // 16-row output tiles of the head dim
  constexpr int DP = NC * 32 + 8;      // padded K row in LDS
  constexpr int VROWS = NDT * 16;
  constexpr int NT = NW * 64;
  __shared__ bf16 Ks[KB][DP];
  __shared__ bf16 Vt[VROWS][KB + 8];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t bh = blockIdx.y, b = bh / a.H, h = bh - b * a.H;
  const int64_t qbase = (int64_t)blockIdx.x * 16 * NW + wave * 16;
  const int64_t qi = qbase + l16;
  const bool qvalid = qi < a.Sq;
  const int z = blockIdx.z;
  const int64_t kbeg = (int64_t)z * a.kchunk;
  const int64_t kend = std::min(a.Sk, kbeg + a.kchunk);

  // Q^T fragments (B-operand): lane holds q[qi][c*32 + 8*lg .. +7].
  bf16x8 qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d0 = c * 32 + lg * 8;
    qf[c] = (qvalid && d0 < DH) ? load8(a.q + b * a.q_bs + qi * a.q_rs + h * a.q_hs + d0) : zero8();
  }

  f32x4 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int64_t kb = kbeg; kb < kend; kb += KB) {
    // ---- stage K (row-major) and V (transposed) for keys kb .. kb+31
    for (int c = tid; c < KB * (DH / 8); c += NT) {
      const int key = c / (DH / 8), d0 = (c % (DH / 8)) * 8;
      const int64_t kk = kb + key;
      bf16x8 kv = zero8(), vv = zero8();
      if (kk < kend) {
        if (kk < a.sk0) {
          kv = load8(a.k0 + b * a.k0_bs + kk * a.k0_rs + h * a.k0_hs + d0);
          vv = load8(a.v0 + b * a.v0_bs + kk * a.v0_rs + h * a.v0_hs + d0);
        } else {
          const int64_t k1i = kk - a.sk0;
          kv = load8(a.k1 + b * a.k1_bs + k1i * a.k1_rs + h * a.k1_hs + d0);
          vv = load8(a.v1 + b * a.v1_bs + k1i * a.v1_rs + h * a.v1_hs + d0);
        }
      }
      *reinterpret_cast<bf16x8*>(&Ks[key][d0]) = kv;
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[d0 + e][key] = vv[e];
    }
    __syncthreads();

    // ---- S^T = K Q^T for the two 16-key sub-tiles
    f32x4 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sacc[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d0 = c * 32 + lg * 8;
        const bf16x8 kfr = (d0 < DH) ? *reinterpret_cast<const bf16x8*>(&Ks[kt * 16 + l16][d0]) : zero8();
        sacc[kt] = mfma16(kfr, qf[c], sacc[kt]);
      }
    }

    // ---- scale, mask, online softmax (per lane: one query, 8 keys)
    float s[2][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t kk = kb + kt * 16 + lg * 4 + e;
        float v = sacc[kt][e] * a.scale_log2;
        if (kk >= kend) {
          v = -INFINITY;
        } else if (a.mask_kind != FAM_MASK_NONE && qvalid) {
          const int64_t mi = b * a.mbs + h * a.mhs + qi * a.mqs + kk;
          if (a.mask_kind == FAM_MASK_BOOL) {
            if (!reinterpret_cast<const uint8_t*>(a.mask)[mi]) v = -INFINITY;
          } else if (a.mask_kind == FAM_MASK_ADD_F32) {
            v += reinterpret_cast<const float*>(a.mask)[mi] * 1.4426950408889634f;
          } else {
            v += to_f(reinterpret_cast<const bf16*>(a.mask)[mi]) * 1.4426950408889634f;
          }
        }
        s[kt][e] = v;
        mloc = fmaxf(mloc, v);
      }
    const float m_new = fmaxf(m_run, group4_max(mloc));
    float psum = 0.f;
    bf16x8 pf;
    if (m_new == -INFINITY) {
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[j] = (bf16)0.0f;
    } else {
      const float alpha = exp2f(m_run - m_new);  // m_run = -inf -> 0
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = exp2f(s[kt][e] - m_new);
          psum += p;
          pf[kt * 4 + e] = to_bf(p);
        }
      l_run = l_run * alpha + group4_sum(psum);
#pragma unroll
      for (int t = 0; t < NDT; ++t) oacc[t] *= alpha;
      m_run = m_new;
    }

    // ---- O^T += V^T P^T
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const int d = t * 16 + l16;
      bf16x8 vfr;
      if (d < DH) {
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(&Vt[d][lg * 4]);
        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(&Vt[d][16 + lg * 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) { vfr[e] = lo[e]; vfr[4 + e] = hi[e]; }
      } else {
        vfr = zero8();
      }
      oacc[t] = mfma16(vfr, pf, oacc[t]);
    }
    __syncthreads();
  }

  // lane owns O[qi][t*16 + 4*lg + e]
  if (a.splits > 1) {
    const int64_t nqt = gridDim.x;
    const int64_t tile = bh * nqt + blockIdx.x;
    const int64_t rowz = ((int64_t)z * gridDim.y + bh) * a.sq_pad + qi;  // (split, b*h, q)
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const int d0 = t * 16 + lg * 4;
      if (d0 < DH) *reinterpret_cast<f32x4*>(a.opart + rowz * DH + d0) = oacc[t];
    }
    if (lg == 0) { a.mlpart[rowz * 2] = m_run; a.mlpart[rowz * 2 + 1] = l_run; }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&a.cnt[tile], 1u) == (unsigned)(a.splits - 1));
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    float mx = -INFINITY;
    for (int zz = 0; zz < a.splits; ++zz) {
      const int64_t r = ((int64_t)zz * gridDim.y + bh) * a.sq_pad + qi;
      mx = fmaxf(mx, *reinterpret_cast<const volatile float*>(a.mlpart + r * 2));
    }
    l_run = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (mx != -INFINITY) {
      for (int zz = 0; zz < a.splits; ++zz) {
        const int64_t r = ((int64_t)zz * gridDim.y + bh) * a.sq_pad + qi;
        const float mz = *reinterpret_cast<const volatile float*>(a.mlpart + r * 2);
        const float lz = *reinterpret_cast<const volatile float*>(a.mlpart + r * 2 + 1);
        const float w = exp2f(mz - mx);  // mz = -inf -> 0
        l_run += lz * w;
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const int d0 = t * 16 + lg * 4;
          if (d0 < DH) {
            const f32x4 p = *reinterpret_cast<const volatile f32x4*>(a.opart + r * DH + d0);
            oacc[t] += p * w;
          }
        }
      }
    }
    if (tid == 0) atomicExch(&a.cnt[tile], 0u);
  }

  if (!qvalid) return;
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  bf16* orow = a.o + b * a.o_bs + qi * a.o_rs + h * a.o_hs;
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    const int d0 = t * 16 + lg * 4;
    if (d0 < DH) {
      bf16x4 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = to_bf(oacc[t][e] * inv);
      *reinterpret_cast<bf16x4*>(orow + d0) = ov;
    }
  }
}

static int pick_nw(int64_t sq) { return sq <= 16 ? 1 : (sq <= 32 ? 2 : 4); }

static int64_t rup(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

static int auto_splits(int64_t tiles, int64_t sk) {
  const int64_t nkb = (sk + KB - 1) / KB;
  if (tiles >= 256 || nkb < 4) return 1;
  int64_t s = (512 + tiles - 1) / tiles;
  s = std::min<int64_t>(s, nkb / 2);
  s = std::min<int64_t>(s, 32);
  return (int)std::max<int64_t>(s, 1);
}

static int resolve_splits(int64_t B, int64_t H, int64_t sq, int64_t sk, int req) {
  const int nw = pick_nw(sq);
  const int64_t tiles = rup(sq, 16 * nw) / (16 * nw) * B * H;
  int s = req > 0 ? req : auto_splits(tiles, sk);
  const int64_t nkb = std::max<int64_t>((sk + KB - 1) / KB, 1);
  if (s > nkb) s = (int)nkb;
  return s;
}


}  // namespace fam

using namespace fam;

extern "C" int64_t fam_attention_workspace_bytes(int64_t batch, int64_t heads, int64_t sq, int64_t sk,
                                                 int64_t head_dim, int num_splits) {
  if (batch <= 0 || heads <= 0 || sq <= 0 || sk <= 0 || head_dim <= 0) return 0;
  const int s = resolve_splits(batch, heads, sq, sk, num_splits);
  if (s <= 1) return 0;
  const int64_t rows = (int64_t)s * batch * heads * rup(sq, 64);
  return FAM_WS_COUNTER_BYTES + rows * head_dim * 4 + rows * 2 * 4;
}

template <int DH>
static void launch_dh(const AttnArgs& a, int nw, dim3 grid, hipStream_t s) {
  if (nw == 1) hipLaunchKernelGGL((attn_kernel<DH, 1>), grid, dim3(64), 0, s, a);
  else if (nw == 2) hipLaunchKernelGGL((attn_kernel<DH, 2>), grid, dim3(128), 0, s, a);
  else hipLaunchKernelGGL((attn_kernel<DH, 4>), grid, dim3(256), 0, s, a);
}

extern "C" int fam_attention(const fam_attn_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_attention: null descriptor");
  const int64_t Dh = d->head_dim;
  FAM_REQUIRE(Dh == 8 || Dh == 16 || Dh == 32 || Dh == 64 || Dh == 128, FAM_ERR_UNSUPPORTED,
              "fam_attention: head_dim must be 8, 16, 32, 64 or 128 (got %lld)", (long long)Dh);
  FAM_REQUIRE(d->batch >= 0 && d->heads >= 1 && d->sq >= 0 && d->sk0 >= 0 && d->sk1 >= 0, FAM_ERR_INVALID_ARG,
              "fam_attention: negative size");
  FAM_REQUIRE(d->q && d->o && (d->sk0 == 0 || (d->k0 && d->v0)) && (d->sk1 == 0 || (d->k1 && d->v1)),
              FAM_ERR_INVALID_ARG, "fam_attention: missing tensor pointer");
  const int64_t strides[] = {d->q_bs, d->q_rs, d->q_hs, d->k0_bs, d->k0_rs, d->k0_hs, d->v0_bs, d->v0_rs, d->v0_hs,
                             d->k1_bs, d->k1_rs, d->k1_hs, d->v1_bs, d->v1_rs, d->v1_hs, d->o_bs, d->o_rs, d->o_hs};
  for (int64_t st : strides) {
    FAM_REQUIRE(st % 8 == 0, FAM_ERR_INVALID_ARG, "fam_attention: strides must be multiples of 8 elements");
  }
  FAM_REQUIRE(fam_host::aligned16(d->q) && fam_host::aligned16(d->o) && fam_host::aligned16(d->k0) &&
                  fam_host::aligned16(d->v0) && fam_host::aligned16(d->k1) && fam_host::aligned16(d->v1),
              FAM_ERR_INVALID_ARG, "fam_attention: base pointers must be 16-byte aligned");
  FAM_REQUIRE(d->mask_kind >= FAM_MASK_NONE && d->mask_kind <= FAM_MASK_ADD_BF16, FAM_ERR_INVALID_ARG,
              "fam_attention: unknown mask kind %d", d->mask_kind);
  FAM_REQUIRE(d->mask_kind == FAM_MASK_NONE || d->mask, FAM_ERR_INVALID_ARG, "fam_attention: mask kind without mask");
  FAM_REQUIRE(d->num_splits >= 0 && d->num_splits <= 64, FAM_ERR_INVALID_ARG, "fam_attention: num_splits in [0, 64]");
  const int64_t Sk = d->sk0 + d->sk1;
  if (d->batch == 0 || d->sq == 0) return FAM_OK;

  const int nw = pick_nw(d->sq);
  const int splits = Sk > 0 ? resolve_splits(d->batch, d->heads, d->sq, Sk, d->num_splits) : 1;
  AttnArgs a{};
  a.q = (const bf16*)d->q; a.q_bs = d->q_bs; a.q_rs = d->q_rs; a.q_hs = d->q_hs;
  a.k0 = (const bf16*)d->k0; a.k0_bs = d->k0_bs; a.k0_rs = d->k0_rs; a.k0_hs = d->k0_hs;
  a.v0 = (const bf16*)d->v0; a.v0_bs = d->v0_bs; a.v0_rs = d->v0_rs; a.v0_hs = d->v0_hs;
  a.k1 = (const bf16*)d->k1; a.k1_bs = d->k1_bs; a.k1_rs = d->k1_rs; a.k1_hs = d->k1_hs;
  a.v1 = (const bf16*)d->v1; a.v1_bs = d->v1_bs; a.v1_rs = d->v1_rs; a.v1_hs = d->v1_hs;
  a.o = (bf16*)d->o; a.o_bs = d->o_bs; a.o_rs = d->o_rs; a.o_hs = d->o_hs;
  a.H = d->heads; a.Sq = d->sq; a.sk0 = d->sk0; a.Sk = Sk;
  const int64_t nkb = (Sk + KB - 1) / KB;
  a.kchunk = std::max<int64_t>((nkb + splits - 1) / splits, 1) * KB;
  a.scale_log2 = d->scale * 1.4426950408889634f;
  a.mask = d->mask; a.mask_kind = d->mask_kind; a.mbs = d->mask_bs; a.mhs = d->mask_hs; a.mqs = d->mask_qs;
  a.splits = splits;
  a.sq_pad = rup(d->sq, 64);
  if (splits > 1) {
    const int64_t need = fam_attention_workspace_bytes(d->batch, d->heads, d->sq, Sk, Dh, splits);
    FAM_REQUIRE(d->workspace && d->workspace_bytes >= need && fam_host::aligned16(d->workspace), FAM_ERR_WORKSPACE,
                "fam_attention: %d key splits need a 16-byte aligned workspace of %lld bytes (got %lld)", splits,
                (long long)need, (long long)d->workspace_bytes);
    a.cnt = (unsigned*)d->workspace;
    a.opart = (float*)((char*)d->workspace + FAM_WS_COUNTER_BYTES);
    a.mlpart = a.opart + (int64_t)splits * d->batch * d->heads * a.sq_pad * Dh;
  }
  FAM_REQUIRE(d->batch * d->heads <= 65535, FAM_ERR_UNSUPPORTED, "fam_attention: batch*heads must be <= 65535");
  dim3 grid((unsigned)(rup(d->sq, 16 * nw) / (16 * nw)), (unsigned)(d->batch * d->heads), (unsigned)splits);
  FAM_REQUIRE(splits <= 1 || (int64_t)grid.x * grid.y <= FAM_WS_COUNTER_BYTES / 4, FAM_ERR_UNSUPPORTED,
              "fam_attention: %d key splits with %lld tiles exceed the workspace counter area", splits,
              (long long)grid.x * grid.y);
  hipStream_t s = (hipStream_t)stream;
  switch (Dh) {
    case 8: launch_dh<8>(a, nw, grid, s); break;
    case 16: launch_dh<16>(a, nw, grid, s); break;
    case 32: launch_dh<32>(a, nw, grid, s); break;
    case 64: launch_dh<64>(a, nw, grid, s); break;
    default: launch_dh<128>(a, nw, grid, s); break;
  }
  return fam_host::check_launch("fam_attention");
}
