// GEMM with fused row-normalisation prologue and bias/activation/gate/residual epilogue:
//     out[m, n] = epi( sum_k pro(a)[m, k] * w[n, k] + bias[n] )
// w is in nn.Linear layout [N, K] (K contiguous), a is [M, K] (K contiguous).
//
// Tiling (gfx950, wave64, MFMA v_mfma_f32_16x16x32_bf16):
//   * a 256-thread workgroup (4 waves) owns a BM x BN output tile; the waves are laid out
//     WAVES_M x WAVES_N and each computes (BM/WAVES_M) x (BN/WAVES_N) as 16x16 MFMA tiles;
//   * K advances in steps of BK = 64 (two MFMA k-substeps); the A and W tiles of a step
//     are staged through LDS, double-buffered so one barrier per step suffices, and the
//     next step's global loads are issued before the current step's MFMAs;
//   * the weight tile is the MFMA A-operand and the activation tile the B-operand, so a
//     lane ends up owning 4 consecutive output columns of one row (8-byte stores);
//   * the prologue (LayerNorm, optional affine, or AdaLN modulate) is applied while the
//     activation tile is written to LDS, from per-row statistics computed at kernel start;
//   * split-K: grid.z workgroups share a tile; each writes fp32 partials to the workspace,
//     and the last to arrive (agent-scope counter) sums them in split order and runs the
//     epilogue, then resets the counter, so results are deterministic and the workspace
//     needs no clearing between launches.
//
// Algorithmic bytes per launch (HBM roofline numerator): 2*(M*K + N*K + M*N) (+ bias,
// residual, modulation).  At M <= 64 the weight stream dominates (AI ~ M flop/byte).
#include <algorithm>

#include "fam_common.h"

namespace fam {

constexpr int BK = 64;
constexpr int LDS_K = BK + 8;  // padded row (144 B) to spread LDS banks

struct GemmArgs {
  const bf16* a; int64_t lda;
  const bf16* w; int64_t ldw;
  const bf16* bias;
  bf16* out; int64_t ldo;
  int64_t M, N, K;
  const bf16* pw; const bf16* pb;
  const bf16* shift; const bf16* scale; int64_t mbs, mrs;
  float eps;
  int act;
  const bf16* res; int64_t ldr;
  const bf16* gate; int64_t gbs, grs, gns;
  int64_t rpb;
  int split; int64_t kchunk;  // K range of split z: [z*kchunk, min(K, (z+1)*kchunk))
  unsigned* cnt; float* part;
};

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == FAM_ACT_GELU_TANH) return gelu_tanh(v);
  if (act == FAM_ACT_SILU) return silu(v);
  return v;
}

template <int BM, int BN, int WAVES_M, int PRO>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  constexpr int WAVES_N = 4 / WAVES_M;
  constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int CA = BM * 8 / 256;  // 16-byte A chunks per thread per K step
  constexpr int CW = BN * 8 / 256;  // 16-byte W chunks per thread per K step
  static_assert(CA >= 1 && CW >= 1 && FM >= 1 && FN >= 1, "tile too small");

  __shared__ bf16 As[2][BM][LDS_K];
  __shared__ bf16 Ws[2][BN][LDS_K];
  __shared__ float s_mean[BM], s_rstd[BM];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int wm0 = (wave / WAVES_N) * TM, wn0 = (wave % WAVES_N) * TN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int z = blockIdx.z;
  const int64_t kbeg = (int64_t)z * g.kchunk;
  const int64_t kend = min(g.K, kbeg + g.kchunk);

  // ---- prologue statistics: one wave per row, two passes (mean, then centred variance)
  if constexpr (PRO != FAM_PRO_NONE) {
    for (int r = wave; r < BM; r += 4) {
      const int64_t m = m0 + r;
      float mean = 0.f, rstd = 0.f;
      if (m < g.M) {  // wave-uniform
        const bf16* ar = g.a + m * g.lda;
        float s = 0.f;
        for (int64_t c = (int64_t)lane * 8; c < g.K; c += 512) {
          bf16x8 t = load8(ar + c);
#pragma unroll
          for (int e = 0; e < 8; ++e) s += to_f(t[e]);
        }
        mean = wave_sum(s) / (float)g.K;
        float q = 0.f;
        for (int64_t c = (int64_t)lane * 8; c < g.K; c += 512) {
          bf16x8 t = load8(ar + c);
#pragma unroll
          for (int e = 0; e < 8; ++e) { const float d = to_f(t[e]) - mean; q += d * d; }
        }
        rstd = rsqrtf(wave_sum(q) / (float)g.K + g.eps);
      }
      if (lane == 0) { s_mean[r] = mean; s_rstd[r] = rstd; }
    }
    __syncthreads();
  }

  bf16x8 ra[CA], rw[CW];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int p = 0; p < CA; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      const int64_t m = m0 + r, k = k0 + kc;
      ra[p] = (m < g.M && k < kend) ? load8(g.a + m * g.lda + k) : zero8();
    }
#pragma unroll
    for (int p = 0; p < CW; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      const int64_t n = n0 + r, k = k0 + kc;
      rw[p] = (n < g.N && k < kend) ? load8(g.w + n * g.ldw + k) : zero8();
    }
  };
  auto lstore = [&](int buf, int64_t k0) {
#pragma unroll
    for (int p = 0; p < CA; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      bf16x8 v = ra[p];
      if constexpr (PRO != FAM_PRO_NONE) {
        const int64_t m = m0 + r, k = k0 + kc;
        if (m < g.M && k < kend) {
          const float mu = s_mean[r], rs = s_rstd[r];
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (to_f(v[e]) - mu) * rs;
          if constexpr (PRO == FAM_PRO_LAYERNORM) {
            if (g.pw) {
              bf16x8 wv = load8(g.pw + k);
#pragma unroll
              for (int e = 0; e < 8; ++e) o[e] *= to_f(wv[e]);
            }
            if (g.pb) {
              bf16x8 bv = load8(g.pb + k);
#pragma unroll
              for (int e = 0; e < 8; ++e) o[e] += to_f(bv[e]);
            }
          } else {
            const int64_t bi = m / g.rpb, si = m - bi * g.rpb;
            const int64_t off = bi * g.mbs + si * g.mrs + k;
            bf16x8 sh = load8(g.shift + off), sc = load8(g.scale + off);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = o[e] * (1.0f + to_f(sc[e])) + to_f(sh[e]);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = to_bf(o[e]);
        }
      }
      *reinterpret_cast<bf16x8*>(&As[buf][r][kc]) = v;
    }
#pragma unroll
    for (int p = 0; p < CW; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<bf16x8*>(&Ws[buf][r][kc]) = rw[p];
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t niter = (kend > kbeg) ? (kend - kbeg + BK - 1) / BK : 0;
  if (niter > 0) {
    gload(kbeg);
    lstore(0, kbeg);
    __syncthreads();
  }
  for (int64_t it = 0; it < niter; ++it) {
    const int buf = (int)(it & 1);
    const bool more = it + 1 < niter;
    if (more) gload(kbeg + (it + 1) * BK);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 af[FM], wf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const bf16x8*>(&As[buf][wm0 + i * 16 + l16][s * 32 + lg * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j) wf[j] = *reinterpret_cast<const bf16x8*>(&Ws[buf][wn0 + j * 16 + l16][s * 32 + lg * 8]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(wf[j], af[i], acc[i][j]);
    }
    if (more) lstore(buf ^ 1, kbeg + (it + 1) * BK);
    __syncthreads();
  }

  // ---- split-K: publish partials, last arriver reduces in split order
  if (g.split > 1) {
    const int64_t ntile = (int64_t)gridDim.x * gridDim.y;
    const int64_t tile = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    auto pptr = [&](int zz, int i, int j) {
      const int lm = wm0 + i * 16 + l16, ln = wn0 + j * 16 + lg * 4;
      return g.part + (((int64_t)zz * ntile + tile) * BM + lm) * BN + ln;
    };
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) *reinterpret_cast<f32x4*>(pptr(z, i, j)) = acc[i][j];
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(&g.cnt[tile], 1u);
      s_last = (prev == (unsigned)(g.split - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int zz = 0; zz < g.split; ++zz) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const f32x4 p = *reinterpret_cast<const volatile f32x4*>(pptr(zz, i, j));
          acc[i][j] += p;
        }
    }
    if (tid == 0) atomicExch(&g.cnt[tile], 0u);
  }

  // ---- epilogue: bias, activation, gate * value + residual, bf16 store
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t m = m0 + wm0 + i * 16 + l16;
    if (m >= g.M) continue;
    const int64_t bi = m / g.rpb, si = m - bi * g.rpb;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t nb = n0 + wn0 + j * 16 + lg * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t n = nb + e;
        if (n >= g.N) continue;
        float v = acc[i][j][e];
        if (g.bias) v += to_f(g.bias[n]);
        v = apply_act(v, g.act);
        if (g.res) {
          float gt = 1.0f;
          if (g.gate) gt = to_f(g.gate[bi * g.gbs + si * g.grs + n * g.gns]);
          v = to_f(g.res[m * g.ldr + n]) + gt * v;
        }
        g.out[m * g.ldo + n] = to_bf(v);
      }
    }
  }
}

struct Cfg { int bm, bn, wm; };

static Cfg pick_cfg(int64_t M, int64_t N) {
  if (M <= 32) return {32, 64, 1};
  if (M <= 64 || N < 128) return {64, 64, 2};
  return {128, 128, 2};
}

static int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

static int auto_split(int64_t tiles, int64_t K) {
  const int64_t kiter = (K + BK - 1) / BK;
  if (tiles >= 256 || kiter < 4) return 1;
  int64_t s = (512 + tiles - 1) / tiles;
  s = std::min<int64_t>(s, kiter / 2);
  s = std::min<int64_t>(s, 16);
  return (int)std::max<int64_t>(s, 1);
}

}  // namespace fam

using namespace fam;


static int resolve_split(int64_t M, int64_t N, int64_t K, int split_k) {
  const Cfg c = pick_cfg(M, N);
  const int64_t tiles = round_up(M, c.bm) / c.bm * (round_up(N, c.bn) / c.bn);
  int s = split_k > 0 ? split_k : auto_split(tiles, K);
  const int64_t kiter = (K + BK - 1) / BK;
  if (s > kiter) s = (int)std::max<int64_t>(kiter, 1);
  return s;
}

extern "C" int64_t fam_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int split_k) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int s = resolve_split(M, N, K, split_k);
  if (s <= 1) return 0;
  return FAM_WS_COUNTER_BYTES + (int64_t)s * round_up(M, 128) * round_up(N, 128) * 4;
}

template <int BM, int BN, int WM>
static void launch_cfg(const GemmArgs& a, int pro, dim3 grid, hipStream_t s) {
  switch (pro) {
    case FAM_PRO_LAYERNORM: hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, FAM_PRO_LAYERNORM>), grid, dim3(256), 0, s, a); break;
    case FAM_PRO_ADALN: hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, FAM_PRO_ADALN>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, FAM_PRO_NONE>), grid, dim3(256), 0, s, a); break;
  }
}

extern "C" int fam_gemm(const fam_gemm_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_gemm: null descriptor");
  FAM_REQUIRE(d->a && d->w && d->out, FAM_ERR_INVALID_ARG, "fam_gemm: a, w and out must be non-null");
  FAM_REQUIRE(d->M >= 0 && d->N >= 1 && d->K >= 8 && d->K % 8 == 0, FAM_ERR_INVALID_ARG,
              "fam_gemm: need N >= 1 and K a positive multiple of 8 (M=%lld N=%lld K=%lld)", (long long)d->M,
              (long long)d->N, (long long)d->K);
  FAM_REQUIRE(d->lda >= d->K && d->ldw >= d->K && d->lda % 8 == 0 && d->ldw % 8 == 0, FAM_ERR_INVALID_ARG,
              "fam_gemm: lda/ldw must be >= K and multiples of 8");
  FAM_REQUIRE(d->ldo >= d->N, FAM_ERR_INVALID_ARG, "fam_gemm: ldo must be >= N");
  FAM_REQUIRE(fam_host::aligned16(d->a) && fam_host::aligned16(d->w), FAM_ERR_INVALID_ARG,
              "fam_gemm: a and w must be 16-byte aligned");
  FAM_REQUIRE(d->prologue >= FAM_PRO_NONE && d->prologue <= FAM_PRO_ADALN, FAM_ERR_INVALID_ARG,
              "fam_gemm: unknown prologue %d", d->prologue);
  FAM_REQUIRE(d->act >= FAM_ACT_NONE && d->act <= FAM_ACT_SILU, FAM_ERR_INVALID_ARG, "fam_gemm: unknown act %d", d->act);
  if (d->prologue == FAM_PRO_LAYERNORM) {
    FAM_REQUIRE((!d->pro_w || fam_host::aligned16(d->pro_w)) && (!d->pro_b || fam_host::aligned16(d->pro_b)),
                FAM_ERR_INVALID_ARG, "fam_gemm: LayerNorm affine must be 16-byte aligned");
  }
  if (d->prologue == FAM_PRO_ADALN) {
    FAM_REQUIRE(d->pro_shift && d->pro_scale, FAM_ERR_INVALID_ARG, "fam_gemm: AdaLN needs shift and scale");
    FAM_REQUIRE(fam_host::aligned16(d->pro_shift) && fam_host::aligned16(d->pro_scale) && d->pro_mod_bs % 8 == 0 &&
                    d->pro_mod_rs % 8 == 0,
                FAM_ERR_INVALID_ARG, "fam_gemm: AdaLN shift/scale must be 16-byte aligned, strides %% 8 == 0");
  }
  FAM_REQUIRE(d->rows_per_batch >= 1, FAM_ERR_INVALID_ARG, "fam_gemm: rows_per_batch must be >= 1");
  FAM_REQUIRE(!d->gate || d->res, FAM_ERR_INVALID_ARG, "fam_gemm: a gate needs a residual");
  FAM_REQUIRE(d->split_k >= 0 && d->split_k <= 64, FAM_ERR_INVALID_ARG, "fam_gemm: split_k must be in [0, 64]");
  if (d->M == 0) return FAM_OK;

  const Cfg c = pick_cfg(d->M, d->N);
  const int split = resolve_split(d->M, d->N, d->K, d->split_k);
  GemmArgs a{};
  a.a = (const bf16*)d->a; a.lda = d->lda;
  a.w = (const bf16*)d->w; a.ldw = d->ldw;
  a.bias = (const bf16*)d->bias;
  a.out = (bf16*)d->out; a.ldo = d->ldo;
  a.M = d->M; a.N = d->N; a.K = d->K;
  a.pw = (const bf16*)d->pro_w; a.pb = (const bf16*)d->pro_b;
  a.shift = (const bf16*)d->pro_shift; a.scale = (const bf16*)d->pro_scale;
  a.mbs = d->pro_mod_bs; a.mrs = d->pro_mod_rs; a.eps = d->pro_eps;
  a.act = d->act;
  a.res = (const bf16*)d->res; a.ldr = d->ldr;
  a.gate = (const bf16*)d->gate; a.gbs = d->gate_bs; a.grs = d->gate_rs; a.gns = d->gate_ns;
  a.rpb = d->rows_per_batch;
  a.split = split;
  const int64_t kiter = (d->K + BK - 1) / BK;
  a.kchunk = ((kiter + split - 1) / split) * BK;
  if (split > 1) {
    const int64_t need = fam_gemm_workspace_bytes(d->M, d->N, d->K, split);
    FAM_REQUIRE(d->workspace && d->workspace_bytes >= need && fam_host::aligned16(d->workspace), FAM_ERR_WORKSPACE,
                "fam_gemm: split_k=%d needs a 16-byte aligned workspace of %lld bytes (got %lld)", split,
                (long long)need, (long long)d->workspace_bytes);
    a.cnt = (unsigned*)d->workspace;
    a.part = (float*)((char*)d->workspace + FAM_WS_COUNTER_BYTES);
  }
  dim3 grid((unsigned)(round_up(d->N, c.bn) / c.bn), (unsigned)(round_up(d->M, c.bm) / c.bm), (unsigned)split);
  FAM_REQUIRE(split <= 1 || (int64_t)grid.x * grid.y <= FAM_WS_COUNTER_BYTES / 4, FAM_ERR_UNSUPPORTED,
              "fam_gemm: split_k=%d with %lld tiles exceeds the workspace counter area", split,
              (long long)grid.x * grid.y);
  FAM_REQUIRE(grid.y <= 65535 && split <= 65535, FAM_ERR_UNSUPPORTED, "fam_gemm: M too large");
  hipStream_t s = (hipStream_t)stream;
  if (c.bm == 32) launch_cfg<32, 64, 1>(a, d->prologue, grid, s);
  else if (c.bm == 64) launch_cfg<64, 64, 2>(a, d->prologue, grid, s);
  else launch_cfg<128, 128, 2>(a, d->prologue, grid, s);
  return fam_host::check_launch("fam_gemm");
}
