// GEMM with fused row-normalisation prologue and bias/activation/gate/residual epilogue:
//     out[m, n] = epi( sum_k pro(a)[m, k] * w[n, k] + bias[n] )
// w is in nn.Linear layout [N, K] (K contiguous), a is [M, K] (K contiguous).
//
// Kernels chosen by M and shape; none communicates between workgroups (on gfx950 a release /
// acquire fence between workgroups writes back and invalidates the XCD's L2, which costs far
// more than these small products), so every workgroup owns its outputs outright.
//
// skinny_kernel (M <= 64, the 16..64-token action projections): weight streaming.
//   * a workgroup of 8 waves owns 16 output columns for all M rows; the waves split the K
//     range (32-wide MFMA k-steps, contiguous per wave) and each wave issues the loads of its
//     whole weight slice up front, so a workgroup keeps its full 16 x K weight panel in
//     flight at once -- the bytes in flight, not the MFMA rate, bound this regime;
//   * the weight rows are the MFMA A-operand and the activations the B-operand
//     (v_mfma_f32_16x16x32_bf16), read straight from global memory (the activation block is
//     small and L2-resident); the LayerNorm / AdaLN prologue is applied in registers from
//     per-row statistics the waves compute at kernel start while the weights are in flight;
//   * the 8 partial accumulators are summed through LDS in wave order (deterministic), then
//     the epilogue runs one output element per thread.
//   Bytes per launch (HBM roofline numerator): 2*(N*K + M*K + M*N) + bias/residual/modulation.
//
// partial_kernel (M <= 128, used by the fused action expert and the video prefill): split-K without any
// cross-workgroup traffic.  A workgroup of 4 waves owns 16 output columns over one K slice
// and its waves split the slice again (summed through LDS); every weight and activation
// fragment of a wave is loaded before the first MFMA.  The slice length is chosen so that
// >= 256 workgroups stream the weights (on gfx950 the per-CU memory parallelism, not HBM,
// limits a skinny product spread over few CUs) with as few partial planes as possible.  The
// fp32 partials partial[z][m][n] are summed, in split order, by the row kernel that follows
// (fam_rowop), which also runs the epilogue and the next normalisation on whole rows.
//
// big_kernel (M >= 128, no prologue, K % 64 == 0: the video backbone's projections, the
// per-call context K/V, batched throughput points): 256 x 256 down to 64 x 64 tiles fed by
// direct-to-LDS loads; described at its definition.
//
// tiled_kernel (M > 64 outside the big kernel's envelope, e.g. with a normalising prologue):
//   * 256-thread workgroup, BM x BN output tile (64x64 or 128x128), 2x2 waves of 16x16 MFMA
//     tiles, K in steps of 64 through double-buffered LDS, next step's global loads issued
//     before the current step's MFMAs; prologue statistics per tile row at kernel start.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "fam_common.h"

namespace fam {

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
  int out_f32;
  const float* csum;   // FAM_PRO_LN_FOLDED: sum_k w[n, k], fp32 [N]
};

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == FAM_ACT_GELU_TANH) return gelu_tanh(v);
  if (act == FAM_ACT_SILU) return silu(v);
  if (act == FAM_ACT_RELU) return fmaxf(v, 0.f);
  if (act == FAM_ACT_GELU_ERF) return gelu_erf(v);
  return v;
}

// The epilogue operands of one output element (row m < M, column n < N: callers clamp), loaded
// ahead of the product so that their memory round trip overlaps the weight stream.  The loads
// are branch-free and keep the raw bits: an absent operand reads element 0 of the weight matrix
// (a valid address) and epilogue_finish ignores it.  A load under a branch, converted on the
// spot, made the compiler wait for every load issued before it (the weight stream included),
// one memory round trip per operand.
struct EpiIn {
  bf16 bias, gate, resb;
  float resf, csum;
};
__device__ __forceinline__ EpiIn epilogue_load(const GemmArgs& g, int64_t m, int64_t n) {
  const int64_t bi = m / g.rpb, si = m - bi * g.rpb;
  const bool rb = g.res && !g.out_f32, rf = g.res && g.out_f32;
  const float* wf = reinterpret_cast<const float*>(g.w);
  EpiIn e;
  e.bias = (g.bias ? g.bias : g.w)[g.bias ? n : 0];
  e.gate = (g.gate ? g.gate : g.w)[g.gate ? bi * g.gbs + si * g.grs + n * g.gns : 0];
  e.resb = (rb ? g.res : g.w)[rb ? m * g.ldr + n : 0];
  e.resf = (rf ? reinterpret_cast<const float*>(g.res) : wf)[rf ? m * g.ldr + n : 0];
  e.csum = (g.csum ? g.csum : wf)[g.csum ? n : 0];
  return e;
}
__device__ __forceinline__ void epilogue_finish(const GemmArgs& g, int64_t m, int64_t n, float v, const EpiIn& e) {
  v = apply_act(v + (g.bias ? to_f(e.bias) : 0.f), g.act);
  if (g.res) v = (g.out_f32 ? e.resf : to_f(e.resb)) + (g.gate ? to_f(e.gate) : 1.f) * v;
  if (g.out_f32) reinterpret_cast<float*>(g.out)[m * g.ldo + n] = v;
  else g.out[m * g.ldo + n] = to_bf(v);
}

// bias, activation, gate * value + residual, store (bf16 or fp32) for one output element
__device__ __forceinline__ void epilogue_store(const GemmArgs& g, int64_t m, int64_t n, float v) {
  if (g.bias) v += to_f(g.bias[n]);
  v = apply_act(v, g.act);
  if (g.res) {
    const int64_t bi = m / g.rpb, si = m - bi * g.rpb;
    float gt = 1.0f;
    if (g.gate) gt = to_f(g.gate[bi * g.gbs + si * g.grs + n * g.gns]);
    const float r = g.out_f32 ? reinterpret_cast<const float*>(g.res)[m * g.ldr + n] : to_f(g.res[m * g.ldr + n]);
    v = r + gt * v;
  }
  if (g.out_f32) reinterpret_cast<float*>(g.out)[m * g.ldo + n] = v;
  else g.out[m * g.ldo + n] = to_bf(v);
}

// LayerNorm / AdaLN of 8 consecutive elements (row m, columns k..k+7) of the A operand.
template <int PRO>
__device__ __forceinline__ bf16x8 prologue8(const GemmArgs& g, bf16x8 v, int64_t m, int64_t k, float mu, float rs) {
  if constexpr (PRO == FAM_PRO_NONE) {
    return v;
  } else {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (to_f(v[e]) - mu) * rs;
    if constexpr (PRO == FAM_PRO_LAYERNORM) {
      if (g.pw) {
        const bf16x8 wv = load8(g.pw + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= to_f(wv[e]);
      }
      if (g.pb) {
        const bf16x8 bv = load8(g.pb + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += to_f(bv[e]);
      }
    } else {
      const int64_t bi = m / g.rpb, si = m - bi * g.rpb;
      const int64_t off = bi * g.mbs + si * g.mrs + k;
      const bf16x8 sh = load8(g.shift + off), sc = load8(g.scale + off);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = o[e] * (1.0f + to_f(sc[e])) + to_f(sh[e]);
    }
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = to_bf(o[e]);
    return r;
  }
}

// LayerNorm / AdaLN of 8 elements with the per-column vectors already in registers: p0, p1 =
// (weight, bias) for LayerNorm (use flags uw, ub), (shift, scale) for a broadcast AdaLN.
template <int PRO>
__device__ __forceinline__ bf16x8 prologue8_pre(bf16x8 v, float mu, float rs, bf16x8 p0, bf16x8 p1, bool uw, bool ub) {
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (to_f(v[e]) - mu) * rs;
  if constexpr (PRO == FAM_PRO_LAYERNORM) {
    if (uw) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= to_f(p0[e]);
    }
    if (ub) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += to_f(p1[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = o[e] * (1.0f + to_f(p1[e])) + to_f(p0[e]);
  }
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = to_bf(o[e]);
  return r;
}

// Row statistics (mean, rstd) of rows m0 .. m0+rows-1: one wave per row, two passes
// (mean, then centred variance); rows past M get zeros.
__device__ __forceinline__ void row_stats(const GemmArgs& g, int64_t m0, int rows, int wave, int nwaves, int lane,
                                          float* s_mean, float* s_rstd) {
  for (int r = wave; r < rows; r += nwaves) {
    const int64_t m = m0 + r;
    float mean = 0.f, rstd = 0.f;
    if (m < g.M) {  // wave-uniform
      const bf16* ar = g.a + m * g.lda;
      float s = 0.f;
      for (int64_t c = (int64_t)lane * 8; c < g.K; c += 512) {
        const bf16x8 t = load8(ar + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += to_f(t[e]);
      }
      mean = wave_sum(s) / (float)g.K;
      float q = 0.f;
      for (int64_t c = (int64_t)lane * 8; c < g.K; c += 512) {
        const bf16x8 t = load8(ar + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) { const float d = to_f(t[e]) - mean; q += d * d; }
      }
      rstd = rsqrtf(wave_sum(q) / (float)g.K + g.eps);
    }
    if (lane == 0) { s_mean[r] = mean; s_rstd[r] = rstd; }
  }
}

// ---------------------------------------------------------------------------------------
// skinny_kernel: M <= 16*MT rows, 16 output columns per workgroup, NW waves split K into
// contiguous runs of 32-wide k-steps; each wave holds KS k-steps of weights and activations
// in registers at once.  Every load is branch-free (out-of-range lanes load a valid address
// and are zeroed), so the loads of a chunk are issued back to back.  The per-column prologue
// vectors (LayerNorm weight / bias, a broadcast AdaLN's shift / scale) travel with the chunk
// and each thread's epilogue operands (bias, residual, gate) are loaded before the product,
// so a launch waits for one memory round trip instead of three.
//
// FAM_PRO_LN_FOLDED: the product runs on the raw rows; every lane also sums (x - pivot) and
// (x - pivot)^2 of the elements it loaded (pivot = the row's first element, which keeps the
// variance of rows with a large mean well conditioned), off the path into the matrix cores.
// The sums meet in LDS with the accumulators and the epilogue forms
//   rstd * (acc - mean * csum[n]).
template <int MT, int NW, int KS, int PRO>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(GemmArgs g) {
  constexpr int MR = MT * 16;
  constexpr int TPR = NW * 64 / MR;  // threads per row in the statistics pass
  constexpr bool NORM = PRO == FAM_PRO_LAYERNORM || PRO == FAM_PRO_ADALN;   // normalise the A operand
  constexpr bool FOLD = PRO == FAM_PRO_LN_FOLDED;
  static_assert(!FOLD || NW <= 8, "the folded LayerNorm uses the 8-wave variant");
  __shared__ float s_mean[MR], s_rstd[MR];
  __shared__ float s_red[NW][MR][16];
  __shared__ float2 s_st[FOLD ? NW : 1][MR];
  __shared__ float s_piv[MR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t nsub = (g.K + 31) / 32;       // 32-wide k-steps
  const int64_t per = (nsub + NW - 1) / NW;   // k-steps per wave
  const int64_t s_beg = std::min(nsub, (int64_t)wave * per), s_end = std::min(nsub, s_beg + per);
  const bool nok = n0 + l16 < g.N;
  const bf16* wrow = g.w + (nok ? n0 + l16 : 0) * g.ldw;

  f32x4 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // per-column prologue vectors in registers: LayerNorm always, AdaLN when its modulation is
  // one row for all rows (otherwise prologue8 loads it per row)
  const bool pre = PRO == FAM_PRO_LAYERNORM || (PRO == FAM_PRO_ADALN && g.mbs == 0 && g.mrs == 0);
  const bf16* pv0p = PRO == FAM_PRO_LAYERNORM ? g.pw : g.shift;
  const bf16* pv1p = PRO == FAM_PRO_LAYERNORM ? g.pb : g.scale;
  const bool uw = pv0p != nullptr, ub = pv1p != nullptr;

  bf16x8 wf[KS], af[KS][MT], pv0[KS], pv1[KS];
  auto chunk_load = [&](int64_t sb) {
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const int64_t k = (sb + j) * 32 + lg * 8;
      const bool kok = (sb + j < s_end) && k < g.K;
      wf[j] = load8_if(kok && nok, wrow + k, g.w);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int64_t m = i * 16 + l16;
        af[j][i] = load8_if(kok && m < g.M, g.a + m * g.lda + k, g.a);
      }
      if constexpr (NORM) {
        if (pre) {   // wave-uniform
          pv0[j] = load8_if(kok && uw, pv0p + k, g.a);
          pv1[j] = load8_if(kok && ub, pv1p + k, g.a);
        }
      }
    }
  };
  chunk_load(s_beg);  // weights and activations of the first chunk in flight at once
  float piv[MT], s1[MT], s2[MT];
  if constexpr (FOLD) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int64_t m = i * 16 + l16;
      piv[i] = to_f(g.a[(m < g.M ? m : g.M - 1) * g.lda]);
      s1[i] = 0.f;
      s2[i] = 0.f;
    }
  }
  // epilogue operands of this thread's outputs (at most EPT of them); the 16-wave variants
  // (128 registers per lane) load them in the epilogue instead, as they would spill
  constexpr int EPT = (MR * 16 + NW * 64 - 1) / (NW * 64);
  constexpr bool EPRE = NW <= 8;
  EpiIn ep[EPT];
  auto ep_load = [&]() {
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int t = tid + u * NW * 64, mr = t >> 4;
      const int64_t n = n0 + (t & 15);
      // (outputs past M or N are never stored: their operands are those of a valid element)
      ep[u] = epilogue_load(g, std::min((int64_t)mr, g.M - 1), std::min(n, g.N - 1));
    }
  };
  if constexpr (EPRE) ep_load();
  // keep the scheduler from sinking those loads next to their first use (it would, to save
  // registers, and each k-step would then pay a full memory round trip)
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (NORM) {
    // one pass over each row: sums about the row's first element (a shared pivot keeps the
    // difference of large sums well conditioned), reduced over the TPR lanes of the row
    const int r = tid / TPR, t = tid % TPR;
    const bool rok = r < g.M;
    const bf16* ar = g.a + (rok ? r : 0) * g.lda;
    const float pivot = to_f(ar[0]);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll 8
    for (int64_t c = (int64_t)t * 8; c < g.K; c += TPR * 8) {
      const bf16x8 v = load8(ar + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float d = to_f(v[e]) - pivot; s1 += d; s2 += d * d; }
    }
#pragma unroll
    for (int o = TPR / 2; o >= 1; o >>= 1) {
      s1 += __shfl_xor(s1, o, kWave);
      s2 += __shfl_xor(s2, o, kWave);
    }
    if (t == 0) {
      const float invk = 1.0f / (float)g.K;
      const float dm = s1 * invk;
      const float var = fmaxf(s2 * invk - dm * dm, 0.f);
      s_mean[r] = rok ? pivot + dm : 0.f;
      s_rstd[r] = rok ? rsqrtf(var + g.eps) : 0.f;
    }
    __syncthreads();
  }

  for (int64_t sb = s_beg; sb < s_end; sb += KS) {
    if (sb != s_beg) {
      chunk_load(sb);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < KS; ++j) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        bf16x8 a = af[j][i];
        if constexpr (NORM) {
          // rows past M normalise to finite values that only reach their own (unstored)
          // outputs; k past K meets zero weights
          const int64_t m = i * 16 + l16;
          if (pre) {
            a = prologue8_pre<PRO>(a, s_mean[m], s_rstd[m], pv0[j], pv1[j], uw, ub);
          } else {
            const int64_t k = std::min((sb + j) * 32 + lg * 8, g.K - 8);
            a = prologue8<PRO>(g, a, std::min(m, g.M - 1), k, s_mean[m], s_rstd[m]);
          }
        }
        acc[i] = mfma16(wf[j], a, acc[i]);
      }
    }
    if constexpr (FOLD) {
      // row sums of this chunk (k past the wave's range or K was loaded as zeros: skipped)
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const bool kok = (sb + j < s_end) && (sb + j) * 32 + lg * 8 < g.K;
        if (!kok) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = to_f(af[j][i][e]) - piv[i];
            s1[i] += d;
            s2[i] += d * d;
          }
      }
    }
  }
  if constexpr (FOLD) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      s1[i] = group4_sum(s1[i]);
      s2[i] = group4_sum(s2[i]);
      if (lg == 0) {
        s_st[wave][i * 16 + l16] = make_float2(s1[i], s2[i]);
        if (wave == 0) s_piv[i * 16 + l16] = piv[i];
      }
    }
  }

  // lane holds out[m = i*16 + l16][n = n0 + 4*lg + e]; reduce the waves in order
#pragma unroll
  for (int i = 0; i < MT; ++i) *reinterpret_cast<f32x4*>(&s_red[wave][i * 16 + l16][lg * 4]) = acc[i];
  __syncthreads();
  if constexpr (EPRE) {
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int t = tid + u * NW * 64, mr = t >> 4, nc = t & 15;
      const int64_t n = n0 + nc;
      if (t >= MR * 16 || mr >= g.M || n >= g.N) continue;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += s_red[w][mr][nc];
      if constexpr (FOLD) {
        float t1 = 0.f, t2 = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) { t1 += s_st[w][mr].x; t2 += s_st[w][mr].y; }
        const float invk = 1.0f / (float)g.K;
        const float dm = t1 * invk;
        const float rstd = rsqrtf(fmaxf(t2 * invk - dm * dm, 0.f) + g.eps);
        v = rstd * (v - (s_piv[mr] + dm) * (g.csum ? ep[u].csum : 0.f));
      }
      epilogue_finish(g, mr, n, v, ep[u]);
    }
    return;
  }
  for (int t = tid; t < MR * 16; t += NW * 64) {
    const int mr = t >> 4, nc = t & 15;
    const int64_t n = n0 + nc;
    if (mr >= g.M || n >= g.N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += s_red[w][mr][nc];
    epilogue_store(g, mr, n, v);
  }
}

// ---------------------------------------------------------------------------------------
// partial_kernel: MT m-tiles (M <= 16*MT).  A workgroup owns 16 output columns over one K
// slice of 4*32*STEPS; each of its 4 waves takes a quarter of the slice with every load
// (STEPS weight fragments, MT*STEPS activation fragments) issued before the first MFMA, and
// the 4 wave accumulators are summed through LDS in wave order.  The product is computed
// transposed, D = W A^T, so a lane ends with 4 consecutive columns of one row: one 16-byte
// store per m-tile.
struct PartArgs {
  const bf16* a; int64_t lda;
  const bf16* w; int64_t ldw;
  float* part;               // [splits][M][N]
  int64_t M, N, K;
  // partial_stream_kernel with one split: bf16(sum + bias) into out [M][ldo] instead of a plane
  const bf16* bias;
  bf16* out; int64_t ldo;
};

template <int MT, int STEPS>
__global__ __launch_bounds__(256) void partial_kernel(PartArgs g) {
  __shared__ f32x4 red[4][MT][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t z = blockIdx.y;
  const int64_t kw = z * (4 * 32 * STEPS) + (int64_t)wave * (32 * STEPS) + lg * 8;  // this lane's first k

  // Phase 1: raw loads from clamped (always valid) addresses, nothing else, so the compiler
  // cannot put a wait between them.  Rows past N or M only produce outputs that are never
  // stored; k past K is zeroed on the activation side after the loads.
  const int64_t wn = n0 + l16;
  const bf16* wp = g.w + (wn < g.N ? wn : 0) * g.ldw;
  bf16x8 wf[STEPS], af[MT][STEPS];
  bool kok[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int64_t k = kw + s * 32;
    kok[s] = k < g.K;
    wf[s] = load8(kok[s] ? wp + k : g.w);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int64_t m = t * 16 + l16;
    const bf16* ap = g.a + (m < g.M ? m : 0) * g.lda;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) af[t][s] = load8(kok[s] ? ap + kw + s * 32 : g.a);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
      if (!kok[s]) af[t][s] = zero8();

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) acc[t] = mfma16(wf[s], af[t][s], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  // wave t sums m-tile t over the 4 waves in order and stores it
  for (int t = wave; t < MT; t += 4) {
    const f32x4 v = ((red[0][t][lane] + red[1][t][lane]) + red[2][t][lane]) + red[3][t][lane];
    const int64_t m = t * 16 + l16;            // D[col = 4*lg + e][row = l16]
    const int64_t n = n0 + lg * 4;
    if (m >= g.M) continue;
    float* dst = g.part + (z * g.M + m) * g.N + n;
    if ((g.N & 3) == 0) {
      if (n < g.N) *reinterpret_cast<f32x4*>(dst) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < g.N) dst[e] = v[e];
    }
  }
}

// ---------------------------------------------------------------------------------------
// partial_wide_kernel (64 < M <= 128: the video prefill's 98-token projections; M <= 64 with
// two strips for the large action projections, see partial_plan): the same
// split-K partials, but a workgroup of NWV waves owns 16 NWV output columns (16 per wave)
// over one K slice of 512, and the slice of every activation row is staged once in LDS with
// direct global->LDS loads (one 1 KB row per wave instruction: lane j lands at the row start
// + 16 j) and read by all the waves, which divides the activation re-reads of a 16-column
// workgroup by NWV.
// Each wave streams its own 16 x 512 weight panel into registers; every load is issued before
// the first MFMA.  Rows past M and k past K read finite data that only reaches unstored
// outputs or meets zero weights.
template <int MT, int NWV>
__global__ __launch_bounds__(NWV * 64) void partial_wide_kernel(PartArgs g) {
  constexpr int KSW = 16, KS = 32 * KSW;   // 32-wide k-steps per slice, slice length
  constexpr int PITCH = KS + 16;           // bf16; a 32-byte pad: the 16-byte B-fragment reads of
                                           // a half-wave (16 rows x 2 chunks) hit distinct banks
  __shared__ __attribute__((aligned(16))) bf16 As[MT * 16 * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * (16 * NWV) + wave * 16;
  const int64_t k0 = (int64_t)blockIdx.y * KS;
  const int M = (int)g.M;

  // activation slice: wave w stages rows w, w + 4, ...; k past K re-reads the row's first 8
  const int64_t ka = k0 + lane * 8;
  const int64_t kc = ka + 8 <= g.K ? ka : 0;
  for (int r = wave; r < M; r += NWV)
    __builtin_amdgcn_global_load_lds((const void*)(g.a + (int64_t)r * g.lda + kc),
                                     (__attribute__((address_space(3))) void*)&As[r * PITCH], 16, 0, 0);
  // this wave's weight panel
  const int64_t wn = n0 + l16;
  const bf16* wp = g.w + (wn < g.N ? wn : 0) * g.ldw;
  bf16x8 wf[KSW];
#pragma unroll
  for (int s = 0; s < KSW; ++s) {
    const int64_t k = k0 + s * 32 + lg * 8;
    wf[s] = load8_if(k < g.K, wp + k, g.w);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KSW; ++s)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(&As[(t * 16 + l16) * PITCH + s * 32 + lg * 8]);
      acc[t] = mfma16(wf[s], b, acc[t]);   // D[col n0 + 4 lg + e][row t*16 + l16]
    }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int64_t m = t * 16 + l16;
    const int64_t n = n0 + lg * 4;
    if (m >= M) continue;
    float* dst = g.part + ((int64_t)blockIdx.y * g.M + m) * g.N + n;
    if ((g.N & 3) == 0) {
      if (n < g.N) *reinterpret_cast<f32x4*>(dst) = acc[t];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < g.N) dst[e] = acc[t][e];
    }
  }
}

// ---------------------------------------------------------------------------------------
// partial_stream_kernel (64 < M <= 144, long K ranges): a workgroup of NWV (8 or 4) waves owns
// 16 NWV output columns (16 per wave) over kper = C x 256 of K and walks it in 256-wide chunks.
// While the MFMAs of chunk c run, the next chunk is already in flight: each wave's 16 x 256
// weight panel in registers, and the activation chunk (M rows x 512 B) by direct-to-LDS buffer
// loads into the other of two LDS slots -- no register staging and no LDS stores by the waves.
// A staged row's 16-byte units are XOR-swizzled (unit u of row r at u ^ (r & 15)), so the
// B-fragment reads of 16 rows hit 16 distinct bank groups without padding, and a load
// instruction (2 rows x 512 B, lane j -> row + j / 32, slot j % 32) just fetches the unit that
// belongs in its slot.  Loads go through buffer descriptors: k past the range (and the whole
// weight prefetch after the last chunk) reads zeros without a select on the loaded value, and
// activation rows past M read zeros; activation units past K hold the row's next values, which
// only meet zero weights.  Inside a chunk the fragments of k-step s + 1 are read from LDS while
// the MFMAs of step s run.  Rows past M (M odd: up to one) only reach output rows that are
// never stored.  The partial planes are written with non-temporal stores: the row kernel that
// follows reads them from beyond this XCD's L2 either way, and the L2 is not left holding them.
template <int MT, int NWV>
__global__ __launch_bounds__(NWV * 64) void partial_stream_kernel(PartArgs g, int kper) {
  constexpr int KS = 256, KSW = KS / 32;
  constexpr uint32_t kOob = 0x80000000u;   // beyond every descriptor's range (checked on the host)
  __shared__ __attribute__((aligned(1024))) bf16 As[2][MT * 16 * KS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int M = (int)g.M, K = (int)g.K, N = (int)g.N;
  const int nb0 = blockIdx.x * (16 * NWV), n0 = nb0 + wave * 16;
  const int kb = blockIdx.y * kper;
  const int ke = min(K, kb + kper);
  // descriptors over this workgroup's <= 16 NWV weight rows and the <= 144 activation rows:
  // the host requires M * lda * 2 < 2^31 and 128 * ldw * 2 < 2^31, so both ranges stay below
  // kOob and every out-of-range offset reads zero
  const int nrows = min(16 * NWV, N - nb0);
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(g.w + (int64_t)nb0 * g.ldw, (uint32_t)(nrows * g.ldw * 2));
  const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(g.a, (uint32_t)(g.M * g.lda * 2));
  const int lr = wave * 16 + l16;
  const uint32_t wrow = (uint32_t)((lr < nrows ? lr : 0) * g.ldw) * 2u;
  // activation staging: wave w loads row pairs w, w + NWV, ...; lane j's row and unit
  const int npairs = (M + 1) / 2, sr = lane >> 5;
  const uint32_t lda2 = (uint32_t)g.lda * 2u;
  auto issueA = [&](int k0, int buf) {
    for (int p = wv; p < npairs; p += NWV) {
      // (row & 15) of row 2p + sr is (2p & 15) + sr: the pair's part of the swizzle goes with p
      const uint32_t sw = (uint32_t)((lane & 31) ^ (((2 * p) & 15) + sr)) * 16u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (__attribute__((address_space(3))) void*)&As[buf][2 * p * KS], 16,
                                               (uint32_t)(2 * p + sr) * lda2 + (uint32_t)k0 * 2u + sw, 0, 0, 0);
    }
  };
  bf16x8 wc[KSW], wx[KSW];
  auto loadW = [&](int k0, int klim, bf16x8* wf) {
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      const int k = k0 + s * 32 + lg * 8;
      wf[s] = buffer_load8(wrs, k < klim ? wrow + (uint32_t)k * 2u : kOob);
    }
  };
  issueA(kb, 0);
  loadW(kb, K, wc);
  __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
  __syncthreads();
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = kb, c = 0; k0 < ke; k0 += KS, ++c) {
    const int buf = c & 1;
    const int klim = k0 + KS < ke ? K : 0;   // 0: past the last chunk, every offset is out of range
    if (k0 + KS < ke) issueA(k0 + KS, buf ^ 1);   // that slot was released by the last barrier
    loadW(k0 + KS, klim, wx);
    __builtin_amdgcn_sched_barrier(0);
    const bf16* Ab = As[buf];
    bf16x8 bc[MT], bn[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
      bc[t] = *reinterpret_cast<const bf16x8*>(&Ab[(t * 16 + l16) * KS + ((lg ^ l16) * 8)]);
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      if (s + 1 < KSW) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
          bn[t] = *reinterpret_cast<const bf16x8*>(&Ab[(t * 16 + l16) * KS + ((((s + 1) * 4 + lg) ^ l16) * 8)]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = mfma16(wc[s], bc[t], acc[t]);   // D[col n0 + 4 lg + e][row t*16 + l16]
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < MT; ++t) bc[t] = bn[t];
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // chunk c + 1's activations and weights landed, slot read
    __syncthreads();
#pragma unroll
    for (int s = 0; s < KSW; ++s) wc[s] = wx[s];
  }
  if (g.out != nullptr) {
    // one split (fam_gemm): the finished bf16 row segment with its bias, as nn.Linear rounds it
    // (N % 4 == 0 here)
    const int n = n0 + lg * 4;
    const int nc = n < N ? n : 0;
    bf16x4 bv = *reinterpret_cast<const bf16x4*>(g.bias + nc);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 16 + l16;
      if (m >= M || n >= N) continue;
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = to_bf(acc[t][e] + to_f(bv[e]));
      *reinterpret_cast<bf16x4*>(g.out + (int64_t)m * g.ldo + n) = o;
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = t * 16 + l16, n = n0 + lg * 4;
    if (m >= M) continue;
    float* dst = g.part + ((int64_t)blockIdx.y * g.M + m) * g.N + n;
    if ((N & 3) == 0) {
      if (n < N) __builtin_nontemporal_store(acc[t], reinterpret_cast<f32x4*>(dst));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) __builtin_nontemporal_store(acc[t][e], dst + e);
    }
  }
}

// ---------------------------------------------------------------------------------------
// final_kernel (fam_gemm_final, M <= 64): the whole K of 16 output columns in one workgroup
// of NW waves, each wave a contiguous quarter/eighth/sixteenth of K with every fragment
// loaded before the first MFMA; the wave accumulators are summed through LDS in wave order
// and the epilogue (bias, activation, bf16 store) runs in the same kernel.  Optionally it
// also writes, per row and per 16-column group, the sum of squares of the stored values:
// the statistics a consumer needs for an RMSNorm over any union of column groups.
struct FinalArgs {
  const bf16* a; int64_t lda;
  const bf16* w; int64_t ldw;
  const bf16* bias; int act;
  bf16* out; int64_t ldo;
  float* sumsq;              // [M][ceil(N/16)] or null
  int64_t M, N, K;
};

template <int MT, int NW, int STEPS>
__global__ __launch_bounds__(NW * 64) void final_kernel(FinalArgs g) {
  __shared__ f32x4 red[NW][MT][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t kw = (int64_t)wave * (32 * STEPS) + lg * 8;

  const int64_t wn = n0 + l16;
  const bf16* wp = g.w + (wn < g.N ? wn : 0) * g.ldw;
  bf16x8 wf[STEPS], af[MT][STEPS];
  bool kok[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int64_t k = kw + s * 32;
    kok[s] = k < g.K;
    wf[s] = load8(kok[s] ? wp + k : g.w);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int64_t m = t * 16 + l16;
    const bf16* ap = g.a + (m < g.M ? m : 0) * g.lda;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) af[t][s] = load8(kok[s] ? ap + kw + s * 32 : g.a);
  }
  // the epilogue's bias (4 consecutive columns per lane), loaded with the operands: branch-free
  // (a branch per element made the compiler wait for every load before the next bias load)
  const int64_t nc = n0 + lg * 4;
  const bf16* bsrc = g.bias ? g.bias : g.w;   // a readable address when there is no bias
  float bias[4];
  bf16 braw[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) braw[e] = bsrc[min(nc + e, g.N - 1)];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int e = 0; e < 4; ++e) bias[e] = g.bias ? to_f(braw[e]) : 0.f;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
      if (!kok[s]) af[t][s] = zero8();

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) acc[t] = mfma16(wf[s], af[t][s], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  for (int t = wave; t < MT; t += NW) {
    f32x4 v = red[0][t][lane];
#pragma unroll
    for (int q = 1; q < NW; ++q) v += red[q][t][lane];
    const int64_t m = t * 16 + l16;            // D[col = 4*lg + e][row = l16]
    bf16x4 o;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = v[e] + bias[e];
      if (g.act == FAM_ACT_GELU_TANH) x = gelu_tanh(x);
      else if (g.act == FAM_ACT_SILU) x = silu(x);
      else if (g.act == FAM_ACT_RELU) x = fmaxf(x, 0.f);
      else if (g.act == FAM_ACT_GELU_ERF) x = gelu_erf(x);
      o[e] = to_bf(x);
      const float r = to_f(o[e]);
      ss += (nc + e < g.N) ? r * r : 0.f;
    }
    ss = group4_sum(ss);  // the 16 columns of this group, fixed order
    if (m >= g.M) continue;
    bf16* dst = g.out + m * g.ldo + nc;
    if ((g.N & 3) == 0 && (g.ldo & 3) == 0) {
      if (nc < g.N) *reinterpret_cast<bf16x4*>(dst) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nc + e < g.N) dst[e] = o[e];
    }
    if (g.sumsq && lg == 0) g.sumsq[m * (int64_t)gridDim.x + blockIdx.x] = ss;
  }
}

// ---------------------------------------------------------------------------------------
// tiled_kernel: BM x BN tiles, 4 waves as WAVES_M x WAVES_N.
constexpr int BK = 64;
constexpr int LDS_K = BK + 8;  // padded row (144 B) to spread LDS banks

template <int BM, int BN, int WAVES_M, int PRO>
__global__ __launch_bounds__(256) void tiled_kernel(GemmArgs g) {
  constexpr int WAVES_N = 4 / WAVES_M;
  constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int CA = BM * 8 / 256;  // 16-byte A chunks per thread per K step
  constexpr int CW = BN * 8 / 256;  // 16-byte W chunks per thread per K step
  static_assert(CA >= 1 && CW >= 1 && FM >= 1 && FN >= 1, "tile too small");

  __shared__ bf16 As[2][BM][LDS_K];
  __shared__ bf16 Ws[2][BN][LDS_K];
  __shared__ float s_mean[BM], s_rstd[BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int wm0 = (wave / WAVES_N) * TM, wn0 = (wave % WAVES_N) * TN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

  if constexpr (PRO != FAM_PRO_NONE) {
    row_stats(g, m0, BM, wave, 4, lane, s_mean, s_rstd);
    __syncthreads();
  }

  bf16x8 ra[CA], rw[CW];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int p = 0; p < CA; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      const int64_t m = m0 + r, k = k0 + kc;
      ra[p] = (m < g.M && k < g.K) ? load8(g.a + m * g.lda + k) : zero8();
    }
#pragma unroll
    for (int p = 0; p < CW; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      const int64_t n = n0 + r, k = k0 + kc;
      rw[p] = (n < g.N && k < g.K) ? load8(g.w + n * g.ldw + k) : zero8();
    }
  };
  auto lstore = [&](int buf, int64_t k0) {
#pragma unroll
    for (int p = 0; p < CA; ++p) {
      const int c = tid + 256 * p, r = c >> 3, kc = (c & 7) * 8;
      bf16x8 v = ra[p];
      if constexpr (PRO != FAM_PRO_NONE) {
        const int64_t m = m0 + r, k = k0 + kc;
        if (m < g.M && k < g.K) v = prologue8<PRO>(g, v, m, k, s_mean[r], s_rstd[r]);
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

  const int64_t niter = (g.K + BK - 1) / BK;
  gload(0);
  lstore(0, 0);
  __syncthreads();
  for (int64_t it = 0; it < niter; ++it) {
    const int buf = (int)(it & 1);
    const bool more = it + 1 < niter;
    if (more) gload((it + 1) * BK);
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
    if (more) lstore(buf ^ 1, (it + 1) * BK);
    __syncthreads();
  }

  // lane owns out[m0 + wm0 + i*16 + l16][n0 + wn0 + j*16 + 4*lg + e]
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t m = m0 + wm0 + i * 16 + l16;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t nb = n0 + wn0 + j * 16 + lg * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nb + e < g.N) epilogue_store(g, m, nb + e, acc[i][j][e]);
    }
  }
}

// ---------------------------------------------------------------------------------------
// big_kernel (M >= 128, no prologue, K % 64 == 0): the throughput GEMM of the video backbone
// and of batched action calls.
//   * 256 threads = 2 x 2 waves; a wave owns (16 WFM) x (16 WFN) outputs (up to 128 x 128,
//     256 fp32 accumulators per lane), the workgroup BM x BN = (32 WFM) x (32 WFN):
//     256 x 256, 224 x 256 (M = 1560 splits into 7 such row tiles with 8 padding rows),
//     128 x 128 (two workgroups per CU) or 64 x 64;
//   * K in blocks of 64 through NS LDS slots (two; four for the 64 x 64 tile, whose handful of
//     MFMAs per block cannot cover a block's load latency).  Rows of a slot are 128 bytes (8 chunks of
//     16 B) with chunk c of row r stored at c ^ (r & 7): the 16-byte fragment reads of 8
//     consecutive lanes (8 rows, one chunk) hit 8 distinct bank groups;
//   * the slots are filled by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds): one
//     load writes 1 KB = 8 rows x 128 B, lane l fetching chunk (l % 8) ^ (l / 8) of row l / 8,
//     so the swizzle costs nothing; the descriptors make rows past M or N read zeros (row and
//     k position both go into the vector offset, which the range check covers; the scalar
//     offset is not checked); M0 (LDS slot) is scalar, so a load costs one VALU add;
//   * block b: k-step 0 computes from fragments read during block b - 1 while k-step 1's
//     fragments are read; then one barrier (after which block b + 1 has landed and every wave
//     is done with block b's slot), block b + NS is sent into that slot and k-step 1 computes
//     while k-step 0 of block b + 1 is read.  Loads, fragment reads and MFMAs interleave per
//     MFMA row;
//   * the MFMAs are written as inline assembly with the accumulator tied to an accumulation
//     register ("+a"): with all 256 of them holding accumulators, the compiler's own MFMA
//     form wants a free destination quad and shuffles accumulators through VGPRs every
//     iteration.  Being opaque to the hazard recognizer, the chain is fenced by s_nop before
//     its first and after its last MFMA (the VALU writes of the zero accumulators, the
//     accumulator reads of the epilogue);
//   * workgroups are spread over the 8 XCDs in contiguous task ranges, and a range walks the
//     tile grid column by column in groups of row tiles, so consecutive tiles on one XCD share
//     their weight panel (and row panels) in that XCD's L2;
//   * epilogue: bias, activation, gate * value + residual on 4 consecutive columns per lane,
//     8-byte (bf16) or 16-byte (fp32) stores.
// MFMA operands: A = weight rows (n), B = activation rows (m), so a lane's accumulator holds
// out[m][n .. n + 3] for one m.
#define FAM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ void mfma_acc(f32x4& acc, const bf16x8& w, const bf16x8& a) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(w), "v"(a));
}

// KG = 2 (128 x 128 tiles on a grid of at most one workgroup per CU, an even number of K
// blocks): 8 waves in two K groups of 4; group g takes the K blocks g, g + 2, ... into its own
// two slots, so each SIMD runs two waves although the grid leaves one workgroup per CU; group 1
// then parks its accumulators in LDS for group 0 to add (in a fixed order) before the epilogue.
template <int WFM, int WFN, int KG = 1, int NS = 2>
__global__ __launch_bounds__(256 * KG) void big_kernel(GemmArgs g, int tiles_m, int tiles_n, int vec8, int ksplit, int raw) {
  // the A part of a slot holds BMA >= BM rows, a multiple of 64 (a 224-row tile also loads the
  // next 32 rows, unused: measured 2-4 % faster than 7 loads per wave per block)
  constexpr int BM = 32 * WFM, BN = 32 * WFN, BK = 64, BMA = (BM + 63) / 64 * 64;
  constexpr int SA = BMA * BK, SS = (BMA + BN) * BK;           // elements of a slot's A part, slot
  constexpr int NIA = BMA / 32, NIW = BN / 32, IPW = NIA + NIW;   // 1 KB loads per wave per block
  static_assert(IPW < 64, "vmcnt");
  static_assert(KG == 1 || (KG == 2 && WFM == 4 && WFN == 4), "K groups only on 128 x 128 tiles");
  // NS K slots per group (NS - 1 blocks in flight while one is computed): 2, or 4 for a 64 x 64
  // tile whose grid fits one round at two workgroups per CU (its few MFMAs per block cannot
  // cover a block's load latency; four 16 KB slots still leave room for two workgroups per CU,
  // but not for the three to five a longer grid keeps resident with two).  Later the slots hold
  // the bf16 output tile with its padded rows (and with KG = 2 first group 1's accumulators: 4
  // WFM WFN floats per lane)
  static_assert(NS == 2 || (NS == 4 && WFM == 2 && WFN == 2 && KG == 1), "four slots only on 64 x 64 tiles");
  static_assert((NS - 1) * IPW < 64, "vmcnt");
  constexpr int LDS_SLOTS = KG * NS * SS, LDS_OUT = BM * (BN + 8);
  constexpr int LDS_ELEMS = LDS_SLOTS > LDS_OUT ? LDS_SLOTS : LDS_OUT;
  static_assert(KG == 1 || LDS_ELEMS * 2 >= 4 * (4 * WFM * WFN) * 256, "park area");
  __shared__ __attribute__((aligned(1024))) bf16 sm[LDS_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);   // wave within the K group
  const int kgi = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 8);
  const int l16 = lane & 15, lg = lane >> 4;
  const int wm0 = (wave >> 1) * (16 * WFM), wn0 = (wave & 1) * (16 * WFN);

  // task order: XCD-contiguous ranges (the grid is padded to a multiple of 8; workgroups past
  // the last task exit), split-major (split z covers K blocks [z nb / ksplit, (z+1) nb / ksplit)),
  // then column-major over groups of up to 8 row tiles
  const int ntile = tiles_m * tiles_n, nwg = ntile * ksplit, tpx = (nwg + 7) >> 3;
  const int task_all = (blockIdx.x & 7) * tpx + (blockIdx.x >> 3);
  if (task_all >= nwg) return;   // workgroup-uniform, before any barrier
  const int split = task_all / ntile, task = task_all - split * ntile;
  const int GM = tiles_m < 8 ? tiles_m : 8;
  const int grp = task / (GM * tiles_n), rem = task - grp * (GM * tiles_n);
  const int gm = (tiles_m - grp * GM) < GM ? (tiles_m - grp * GM) : GM;   // rows in this group
  const int tm = grp * GM + rem % gm, tn = rem / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  const int Mi = (int)g.M, Ni = (int)g.N;
  const uint32_t lda2 = (uint32_t)g.lda * 2u, ldw2 = (uint32_t)g.ldw * 2u;
  const auto ra = buffer_rsrc(g.a + (int64_t)m0 * g.lda, (uint32_t)(Mi - m0) * lda2);
  const auto rw = buffer_rsrc(g.w + (int64_t)n0 * g.ldw, (uint32_t)(Ni - n0 < BN ? Ni - n0 : BN) * ldw2);
  const int lr = lane >> 3;
  const uint32_t lc16 = (uint32_t)(((lane & 7) ^ lr) * 16);
  const uint32_t voa = (uint32_t)lr * lda2 + lc16, vow = (uint32_t)lr * ldw2 + lc16;
  const int nball = (int)(g.K / BK);
  const int kb0 = (int)((int64_t)split * nball / ksplit), nbs = (int)((int64_t)(split + 1) * nball / ksplit) - kb0;
  const int nb = nbs / KG;   // blocks of this K group (KG = 2 runs with an even count only)
  // load p of this wave for the group's block blk (of this split) into slot: A rows 8 (wave + 4p)
  // .. + 7 for p < NIA, else W rows 8 (wave + 4 (p - NIA)) .. + 7; blocks past the end re-read
  // the last one (unused).  The group's block j is block KG j + kgi of the split.
  bf16* const smg = sm + kgi * NS * SS;   // this group's slots
  auto dma = [&](int p, int blk, int slot) {
    const uint32_t kb = (uint32_t)(kb0 + KG * (blk < nb ? blk : nb - 1) + kgi) * (BK * 2);
    if (p < NIA) {
      const int r = wave + 4 * p;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, FAM_LDS(smg + slot * SS + r * 512), 16,
                                               voa + (uint32_t)(8 * r) * lda2 + kb, 0, 0, 0);
    } else {
      const int r = wave + 4 * (p - NIA);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, FAM_LDS(smg + slot * SS + SA + r * 512), 16,
                                               vow + (uint32_t)(8 * r) * ldw2 + kb, 0, 0, 0);
    }
  };
  // the fragment of k-step h: row base + l16, chunk 4 h + lg, stored at (4 h + lg) ^ (l16 & 7)
  const int fp0 = (lg ^ (l16 & 7)) << 3, fp1 = ((4 + lg) ^ (l16 & 7)) << 3;
  const bf16* fa = smg + (wm0 + l16) * BK;
  const bf16* fw = smg + SA + (wn0 + l16) * BK;

  f32x4 acc[WFM][WFN];
#pragma unroll
  for (int i = 0; i < WFM; ++i)
#pragma unroll
    for (int j = 0; j < WFN; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      asm volatile("" : "+a"(acc[i][j]));
    }
  asm volatile("s_nop 7");

  bf16x8 a0[WFM], w0[WFN], a1[WFM], w1[WFN];
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
#pragma unroll
    for (int p = 0; p < IPW; ++p) dma(p, sl, sl);
  constexpr int VW0 = (NS - 1) * IPW, VW = (NS - 2) * IPW;
  __builtin_amdgcn_s_waitcnt(0x0070 | (VW0 & 15) | ((VW0 >> 4) << 14));   // vmcnt((NS-1) IPW): block 0
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int i = 0; i < WFM; ++i) a0[i] = *reinterpret_cast<const bf16x8*>(fa + i * 16 * BK + fp0);
#pragma unroll
  for (int j = 0; j < WFN; ++j) w0[j] = *reinterpret_cast<const bf16x8*>(fw + j * 16 * BK + fp0);

  for (int b = 0; b < nb; ++b) {
    const int cur = (b % NS) * SS, nxt = ((b + 1) % NS) * SS;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < WFM; ++i) {
      a1[i] = *reinterpret_cast<const bf16x8*>(fa + cur + i * 16 * BK + fp1);
#pragma unroll
      for (int j = i * WFN / WFM; j < (i + 1) * WFN / WFM; ++j)
        w1[j] = *reinterpret_cast<const bf16x8*>(fw + cur + j * 16 * BK + fp1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < WFN; ++j) mfma_acc(acc[i][j], w0[j], a0[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // vmcnt((NS-2) IPW) lgkmcnt(0): block b + 1 landed (loads complete in order), slot b read
    __builtin_amdgcn_s_waitcnt(0x0070 | (VW & 15) | ((VW >> 4) << 14));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < WFM; ++i) {
#pragma unroll
      for (int p = i * IPW / WFM; p < (i + 1) * IPW / WFM; ++p) dma(p, b + NS, b % NS);
      a0[i] = *reinterpret_cast<const bf16x8*>(fa + nxt + i * 16 * BK + fp0);
#pragma unroll
      for (int j = i * WFN / WFM; j < (i + 1) * WFN / WFM; ++j)
        w0[j] = *reinterpret_cast<const bf16x8*>(fw + nxt + j * 16 * BK + fp0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < WFN; ++j) mfma_acc(acc[i][j], w1[j], a1[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);   // the (unused) loads of blocks nb .. nb + NS - 1 drain before exit
  asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15");
#pragma unroll
  for (int i = 0; i < WFM; ++i)
#pragma unroll
    for (int j = 0; j < WFN; ++j) asm volatile("" : "+a"(acc[i][j]));
  if constexpr (KG == 2) {
    // group 1's accumulators through LDS into group 0's (every wave is past its last fragment
    // read after the first barrier)
    float* park = reinterpret_cast<float*>(sm);
    __syncthreads();
    if (kgi == 1) {
#pragma unroll
      for (int i = 0; i < WFM; ++i)
#pragma unroll
        for (int j = 0; j < WFN; ++j)
          *reinterpret_cast<f32x4*>(park + (((wave * WFM + i) * WFN + j) * 64 + lane) * 4) = acc[i][j];
    }
    __syncthreads();
    if (kgi == 1) {
      // the epilogue's two barriers (pass 1 parks the output tile over the same LDS), without
      // its work; the raw form has none
      if (!raw) {
        __syncthreads();
        __syncthreads();
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < WFM; ++i)
#pragma unroll
      for (int j = 0; j < WFN; ++j) {
        const f32x4 o = *reinterpret_cast<const f32x4*>(park + (((wave * WFM + i) * WFN + j) * 64 + lane) * 4);
        acc[i][j] += o;
      }
  }

  if (raw) {
    // split-K (or fam_gemm_partial's single plane): the raw fp32 sums of this split into plane
    // `split` of out ([ksplit][M][ldo] fp32; bias, activation and residual are the reduction's)
    float* part = reinterpret_cast<float*>(g.out) + (int64_t)split * Mi * g.ldo;
#pragma unroll
    for (int i = 0; i < WFM; ++i) {
      const int m = m0 + wm0 + i * 16 + l16;
      if (m >= Mi) continue;
#pragma unroll
      for (int j = 0; j < WFN; ++j) {
        const int nb4 = n0 + wn0 + j * 16 + lg * 4;
        if (nb4 < Ni) *reinterpret_cast<f32x4*>(part + (int64_t)m * g.ldo + nb4) = acc[i][j];
      }
    }
    return;
  }

  // Epilogue in two passes through LDS (the slots are free now).  Pass 1: every lane adds the
  // bias to its accumulators (lane: out[m][n .. n + 3], one m per lane), rounds to bf16 -- the
  // reference's nn.Linear output -- and parks them in a row-major bf16 tile.  Pass 2: a thread
  // takes VEC consecutive columns of a row (a wave covers 64 VEC contiguous columns) and applies
  // the activation and gate * y + residual on the rounded values, as the reference's separate
  // bf16 ops do, with coalesced residual / gate reads and output stores.  Both passes are
  // compact loops: a per-accumulator copy of a branchy epilogue costs the kernel's instruction
  // cache more than the epilogue's own work, and the stores of a single-round grid are all tail.
  constexpr int EP = BN + 8;   // bf16 row pitch of the parked tile: 16 B of padding per row
  bf16* ot = sm;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < WFN; ++j) {
    const int nl = wn0 + j * 16 + lg * 4, n = n0 + nl;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (g.bias && n < Ni) {
      const bf16x4 b4 = *reinterpret_cast<const bf16x4*>(g.bias + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = to_f(b4[e]);
    }
#pragma unroll
    for (int i = 0; i < WFM; ++i) {
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = to_bf(acc[i][j][e] + bv[e]);
      *reinterpret_cast<bf16x4*>(ot + (wm0 + i * 16 + l16) * EP + nl) = o;
    }
  }
  __syncthreads();
  auto pass2 = [&](auto vec_tag) {
    constexpr int VEC = decltype(vec_tag)::value;
    typedef __bf16 bfv __attribute__((ext_vector_type(VEC)));
    for (int q = tid; q < BM * (BN / VEC); q += 256) {
      const int r = q / (BN / VEC), c = (q - r * (BN / VEC)) * VEC;
      const int m = m0 + r, n = n0 + c;
      if (m >= Mi || n >= Ni) continue;
      const bfv y = *reinterpret_cast<const bfv*>(ot + r * EP + c);
      float v[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = to_f(y[e]);
      if (g.act != FAM_ACT_NONE) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = apply_act(v[e], g.act);
      }
      if (g.res) {
        float gt[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) gt[e] = 1.f;
        if (g.gate) {
          const int rpb = (int)g.rpb, bi = m / rpb, si = m - bi * rpb;
          const bfv gv = *reinterpret_cast<const bfv*>(g.gate + bi * g.gbs + si * g.grs + n);
#pragma unroll
          for (int e = 0; e < VEC; ++e) gt[e] = to_f(gv[e]);
        }
        if (g.out_f32) {
          const float* rp = reinterpret_cast<const float*>(g.res) + (int64_t)m * g.ldr + n;
#pragma unroll
          for (int e4 = 0; e4 < VEC; e4 += 4) {
            const f32x4 r4 = *reinterpret_cast<const f32x4*>(rp + e4);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e4 + e] = r4[e] + gt[e4 + e] * v[e4 + e];
          }
        } else {
          const bfv r8 = *reinterpret_cast<const bfv*>(g.res + (int64_t)m * g.ldr + n);
#pragma unroll
          for (int e = 0; e < VEC; ++e) v[e] = to_f(r8[e]) + gt[e] * v[e];
        }
      }
      if (g.out_f32) {
        float* op = reinterpret_cast<float*>(g.out) + (int64_t)m * g.ldo + n;
#pragma unroll
        for (int e4 = 0; e4 < VEC; e4 += 4)
          *reinterpret_cast<f32x4*>(op + e4) = f32x4{v[e4], v[e4 + 1], v[e4 + 2], v[e4 + 3]};
      } else {
        bfv o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = to_bf(v[e]);
        *reinterpret_cast<bfv*>(g.out + (int64_t)m * g.ldo + n) = o;
      }
    }
  };
  if (vec8) pass2(std::integral_constant<int, 8>{});
  else pass2(std::integral_constant<int, 4>{});
}

static int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

template <int MT, int NW, int KS>
static void launch_skinny(const GemmArgs& a, int pro, hipStream_t s) {
  dim3 grid((unsigned)(round_up(a.N, 16) / 16));
  if constexpr (NW > 8) {
    FAM_LAUNCH((skinny_kernel<MT, NW, KS, FAM_PRO_NONE>), grid, dim3(NW * 64), 0, s, a);
  } else {
    switch (pro) {
      case FAM_PRO_LAYERNORM: FAM_LAUNCH((skinny_kernel<MT, NW, KS, FAM_PRO_LAYERNORM>), grid, dim3(NW * 64), 0, s, a); break;
      case FAM_PRO_ADALN: FAM_LAUNCH((skinny_kernel<MT, NW, KS, FAM_PRO_ADALN>), grid, dim3(NW * 64), 0, s, a); break;
      case FAM_PRO_LN_FOLDED: FAM_LAUNCH((skinny_kernel<MT, NW, KS, FAM_PRO_LN_FOLDED>), grid, dim3(NW * 64), 0, s, a); break;
      default: FAM_LAUNCH((skinny_kernel<MT, NW, KS, FAM_PRO_NONE>), grid, dim3(NW * 64), 0, s, a); break;
    }
  }
}

// 8 waves with 4 k-steps each cover K <= 1024 in one chunk; longer K takes 16 waves with
// 8 k-steps each (K <= 4096 in one chunk), more chunks beyond that.
// The folded LayerNorm always takes 8 waves (its row sums need the registers).
template <int MT>
static void launch_skinny_k(const GemmArgs& a, int pro, hipStream_t s) {
  if (a.K <= 1024 || pro == FAM_PRO_LN_FOLDED) launch_skinny<MT, 8, 4>(a, pro, s);
  else launch_skinny<MT, 16, 8>(a, pro, s);
}

// The big kernel's envelope: no prologue, K % 64 == 0, M >= 128, 32-bit byte offsets into a
// and w (a tile's loads reach up to 256 rows past its first), and a 4-column vector epilogue
// (N % 4 == 0, unit gate column stride, aligned vectors).
static bool big_ok(const fam_gemm_desc* d) {
  const int64_t ob = d->out_f32 ? 16 : 8;
  const auto al = [](const void* p, int64_t b) { return ((uintptr_t)p % (uintptr_t)b) == 0; };
  return d->prologue == FAM_PRO_NONE && d->K % 64 == 0 && d->M >= 128 &&
         (d->M + 256) * d->lda * 2 < ((int64_t)1 << 31) && (d->N + 256) * d->ldw * 2 < ((int64_t)1 << 31) && d->N % 4 == 0 && d->ldo % 4 == 0 && al(d->out, ob) &&
         (!d->bias || al(d->bias, 8)) && (!d->res || (d->ldr % 4 == 0 && al(d->res, ob))) &&
         (!d->gate || (d->gate_ns == 1 && d->gate_bs % 4 == 0 && d->gate_rs % 4 == 0 && al(d->gate, 8)));
}

// raw: fp32 planes without epilogue (always with ksplit > 1)
template <int WFM, int WFN, int KG = 1>
static void launch_big(const GemmArgs& a, hipStream_t s, int ksplit = 1, bool raw = false) {
  const int tm = (int)((a.M + 32 * WFM - 1) / (32 * WFM)), tn = (int)((a.N + 32 * WFN - 1) / (32 * WFN));
  const unsigned grid = (unsigned)(((tm * tn * ksplit + 7) / 8) * 8);
  // 8-column epilogue vectors when every 8-column group of the operands is 16-byte aligned
  const auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const int vec8 = a.N % 8 == 0 && a.ldo % 8 == 0 && al16(a.out) && (!a.res || (a.ldr % 8 == 0 && al16(a.res))) &&
                   (!a.gate || (a.gbs % 8 == 0 && a.grs % 8 == 0 && al16(a.gate)));
  if constexpr (WFM == 2 && WFN == 2 && KG == 1) {
    if ((int64_t)tm * tn * ksplit <= 2 * (int64_t)fam_host::device_cus()) {
      FAM_LAUNCH((big_kernel<2, 2, 1, 4>), dim3(grid), dim3(256), 0, s, a, tm, tn, vec8, ksplit, (int)(raw || ksplit > 1));
      return;
    }
  }
  FAM_LAUNCH((big_kernel<WFM, WFN, KG>), dim3(grid), dim3(256 * KG), 0, s, a, tm, tn, vec8, ksplit,
             (int)(raw || ksplit > 1));
}

// Tile of the big kernel: the candidate with the least estimated time on the busiest CU,
// tiles per CU (ceil(tiles / CUs)) x tile area / efficiency, where the 128 x 128 and 64 x 64
// tiles run 2 and 3 workgroups per CU and the efficiency is the per-CU throughput relative to
// the 256-wide tiles (measured on gfx950: 0.85 for 128 x 128; 64 x 64 is bound by LDS reads,
// four fragments per four MFMAs, about 0.25); ties go to the larger tile.  With an activation
// in the epilogue the 256-wide tiles count at 0.8: their one workgroup per CU evaluates it with
// the matrix cores idle, where one of two 128 x 128 workgroups runs its epilogue while the other
// multiplies (measured with GELU: 1560 x 14336 x 3072 164 -> 144 us, 2048 x 8192 x 2048 81 -> 74
// us on 128 x 128 tiles; without an activation the 256-wide tiles stay ahead on both shapes).
// narrow (fam_gemm only): 128 x 96 tiles (0.8) are a candidate too where the 128 x 128 tiles
// outnumber the CUs -- config 2's 1560 x 3072 products: 312 tiles put two workgroups on 56 CUs,
// 416 narrow ones spread two on 160 CUs with three quarters of the work each.
static void big_plan(int64_t M, int64_t N, int act, int* wfm, int* wfn, bool narrow = false) {
  const int cus = fam_host::device_cus();
  const double big_eff = act == FAM_ACT_NONE ? 1.0 : 0.8;
  const bool n43 = narrow && ((M + 127) / 128) * ((N + 127) / 128) > cus;
  struct C { int fm, fn; double eff; } cands[] = {{8, 8, big_eff}, {7, 8, big_eff}, {4, 4, 0.85}, {4, 3, n43 ? 0.8 : 0.0},
                                                  {2, 2, 0.25}};
  double best = 1e300;
  for (const C& c : cands) {
    if (c.eff <= 0.0) continue;
    const int64_t bm = 32 * c.fm, bn = 32 * c.fn;
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const double t = (double)((tiles + cus - 1) / cus) * (double)(bm * bn) / c.eff;
    if (t < best) { best = t; *wfm = c.fm; *wfn = c.fn; }
  }
}

// 64 x 64 instead of 128 x 128 tiles where the fitted estimate of big_plan_split (below; unsplit:
// ceil(tiles / (CUs occ)) (c0 + 2 bm bn K / rate occ)) is at least 15% lower: a few hundred rows
// (the DiT4DiT backbone's 588 video tokens) give 128 x 128 tiles too few workgroups to fill the
// chip (588 x 2048 x 2048: 80 of 256 CUs), which big_plan's tile-area count does not see.
// 64 x 64 tiles with four K slots (a grid of at most two workgroups per CU, launch_big):
// t = 3.8 us + n W / r_n, W = 2 64 64 K flops per tile, n = ceil(tasks / CUs) <= 2 tiles on the
// busiest CU, r_1 = 2.68 and r_2 = 3.2 TFLOP/s per CU (gfx950: 1024 x 1024 x 1024 6.9 us,
// 1024 x 1024 x 4096 16.3 us at one per CU; 588 x 2048 x 2048 13.8 us, 588 x 2048 x 8192 46.7 us
// with two on 64 CUs).  Returns a negative value for a longer grid (two slots: the fits below).
static double est64_four(int64_t tasks, double kz) {
  const int64_t cus = fam_host::device_cus();
  if (tasks > 2 * cus) return -1.0;
  const int n = tasks > cus ? 2 : 1;
  return 3.8 + (double)n * 2.0 * 64.0 * 64.0 * kz / ((n == 1 ? 2.68 : 3.2) * 1e6);
}

static bool big_prefers_64(int64_t M, int64_t N, int64_t K) {
  const int cus = fam_host::device_cus();
  auto est = [&](int64_t bm, double c0, double rate) {
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bm - 1) / bm);
    return std::ceil((double)tiles / (2.0 * cus)) * (c0 + 2.0 * (double)(bm * bm) * (double)K / (rate * 1e6) * 2.0);
  };
  double e64 = est64_four(((M + 63) / 64) * ((N + 63) / 64), (double)K);
  if (e64 < 0.0) e64 = est(64, 1.0, 3.0);
  return e64 < 0.85 * est(128, 4.0, 5.5);
}

// K split of the big kernel (fam_gemm_ws, and fam_gemm_partial above 144 rows).  Estimated time
// of a tile shape with z splits, a least-squares fit to gfx950 measurements (15 shapes from
// 512 x 6144 x 4096 to 8192^3, every tile, 1-8 splits):
//   t = ceil(tiles z / (CUs occ)) (c0 + 2 bm bn K_z / rate * occ) + [z > 1] z M N 4 B / 12 TB/s
// (K_z = the split's K range; per tile: c0 = 10, 8, 4, 1 us, rate = 6.5, 6.5, 5.5, 3.0 TFLOP/s
// per CU, occ = 1, 1, 2, 2 workgroups per CU for 256x256, 224x256, 128x128, 64x64; the 64 x 64
// tile with four K slots as est64_four).  The cost of
// consuming the planes is added: a row launch that sums them (fam_gemm_ws: about 5 us + the
// bf16 output written at 4 TB/s + z planes read at 8.8 TB/s), or, when a row kernel follows
// anyway (fam_gemm_partial), the reads of the extra planes.  A split (2, 3, 4, 6 or 8 planes, each
// at least 2 blocks of 64 along K, within the workspace) is taken only where this estimate is
// at least 15% below the unsplit one; otherwise *ks = 1 and the tile is big_plan's.
static void big_plan_split(int64_t M, int64_t N, int64_t K, int64_t ws_floats, bool planes_consumed, int* wfm,
                           int* wfn, int* ks) {
  const int cus = fam_host::device_cus();
  struct Fit { int fm, fn; double c0, rate, occ; };
  static const Fit fits[] = {{8, 8, 10.0, 6.5, 1.0}, {7, 8, 8.0, 6.5, 1.0}, {4, 4, 4.0, 5.5, 2.0}, {2, 2, 1.0, 3.0, 2.0}};
  const int64_t nb = K / 64;
  const double mn = (double)M * (double)N;
  auto est = [&](const Fit& f, int z) {
    const int64_t bm = 32 * f.fm, bn = 32 * f.fn;
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const double rounds = std::ceil((double)(tiles * z) / ((double)cus * f.occ));
    const double kz = (double)((nb + z - 1) / z) * 64.0;
    double t = f.fm == 2 ? est64_four(tiles * z, kz) : -1.0;
    if (t < 0.0) t = rounds * (f.c0 + 2.0 * (double)(bm * bn) * kz / (f.rate * 1e6) * f.occ);
    if (z > 1) t += (double)z * mn * 4.0 / 12e6;
    return t;
  };
  double unsplit = 1e300;
  for (const Fit& f : fits) unsplit = std::min(unsplit, est(f, 1));
  double best = 0.85 * unsplit;
  big_plan(M, N, FAM_ACT_NONE, wfm, wfn);
  *ks = 1;
  for (const Fit& f : fits)
    for (int z : {2, 3, 4, 6, 8}) {
      if (nb < 2 * z || (double)z * mn > (double)ws_floats) continue;
      // 64 x 64 splits only where the four-slot estimate holds (the two-slot fit comes from
      // unsplit grids and is optimistic for split ones: 588 x 2048 x 2048 in 3 splits measured
      // 13.8 us of planes against 10.9 estimated)
      if (f.fm == 2 && ((M + 63) / 64) * ((N + 63) / 64) * z > 2 * (int64_t)cus) continue;
      const double consume = planes_consumed ? (double)(z - 1) * mn * 4.0 / 8.8e6
                                             : 5.0 + mn * 2.0 / 4e6 + (double)z * mn * 4.0 / 8.8e6;
      const double t = est(f, z) + consume;
      if (t < best) { best = t; *wfm = f.fm; *wfn = f.fn; *ks = z; }
    }
}

template <int BM, int BN, int WM>
static void launch_tiled(const GemmArgs& a, int pro, hipStream_t s) {
  dim3 grid((unsigned)(round_up(a.N, BN) / BN), (unsigned)(round_up(a.M, BM) / BM));
  switch (pro) {
    case FAM_PRO_LAYERNORM: FAM_LAUNCH((tiled_kernel<BM, BN, WM, FAM_PRO_LAYERNORM>), grid, dim3(256), 0, s, a); break;
    case FAM_PRO_ADALN: FAM_LAUNCH((tiled_kernel<BM, BN, WM, FAM_PRO_ADALN>), grid, dim3(256), 0, s, a); break;
    default: FAM_LAUNCH((tiled_kernel<BM, BN, WM, FAM_PRO_NONE>), grid, dim3(256), 0, s, a); break;
  }
}

}  // namespace fam

using namespace fam;

static void partial_plan(int64_t M, int64_t N, int64_t K, int* steps, int* splits, int* nwv);

// fam_gemm's streaming path: a plain product with a bias (or none) into bf16, 64 < M <= 144, and a
// partial plan of one split of 8-wave workgroups (N >= 32768)
static bool stream_single(const fam_gemm_desc* d) {
  if (d->M <= 64 || d->M > 144 || d->prologue != FAM_PRO_NONE || d->act != FAM_ACT_NONE || d->res || d->gate ||
      d->out_f32 || d->N % 4 || d->ldo % 4 || ((uintptr_t)d->out & 7u) || (d->bias && ((uintptr_t)d->bias & 7u)) ||
      !d->bias || d->M * d->lda * 2 >= (1LL << 31) || d->ldw >= (1LL << 23) || d->N >= (1LL << 31))
    return false;
  int steps, splits, nwv = 8;
  partial_plan(d->M, d->N, d->K, &steps, &splits, &nwv);
  return steps < 0 && splits == 1 && nwv == 8;
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
  FAM_REQUIRE(d->prologue >= FAM_PRO_NONE && d->prologue <= FAM_PRO_LN_FOLDED, FAM_ERR_INVALID_ARG,
              "fam_gemm: unknown prologue %d", d->prologue);
  FAM_REQUIRE(d->act >= FAM_ACT_NONE && d->act <= FAM_ACT_GELU_ERF, FAM_ERR_INVALID_ARG, "fam_gemm: unknown act %d", d->act);
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
  if (d->prologue == FAM_PRO_LN_FOLDED) {
    FAM_REQUIRE(d->pro_w && ((uintptr_t)d->pro_w & 3u) == 0, FAM_ERR_INVALID_ARG,
                "fam_gemm: the folded LayerNorm needs the fp32 column sums of w in pro_w");
    FAM_REQUIRE(d->M <= 64, FAM_ERR_UNSUPPORTED, "fam_gemm: the folded LayerNorm supports M <= 64 (got %lld)",
                (long long)d->M);
  }
  FAM_REQUIRE(d->rows_per_batch >= 1, FAM_ERR_INVALID_ARG, "fam_gemm: rows_per_batch must be >= 1");
  FAM_REQUIRE(!d->gate || d->res, FAM_ERR_INVALID_ARG, "fam_gemm: a gate needs a residual");
  FAM_REQUIRE(d->N <= (int64_t)65535 * 16 && d->M <= (int64_t)65535 * 64, FAM_ERR_UNSUPPORTED, "fam_gemm: too large");
  if (d->M == 0) return FAM_OK;

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
  a.out_f32 = d->out_f32 != 0;
  if (d->prologue == FAM_PRO_LN_FOLDED) {
    a.csum = (const float*)d->pro_w;
    a.pw = nullptr;
  }
  hipStream_t s = (hipStream_t)stream;
  // 64 < M <= 144 rows against N >= 32768 columns (the stacked context K/V of every block): the
  // streaming split-K plan needs no K split there (one round of 128-column workgroups), so it
  // reads the weights once and stores the finished bf16 rows itself
  if (stream_single(d)) {
    int steps, splits, nwv = 8;
    partial_plan(d->M, d->N, d->K, &steps, &splits, &nwv);
    PartArgs pa{(const bf16*)d->a, d->lda, (const bf16*)d->w, d->ldw, nullptr, d->M, d->N, d->K,
                (const bf16*)d->bias, (bf16*)d->out, d->ldo};
    const dim3 grid((unsigned)((d->N + 127) / 128), 1u);
    const int kper = -steps * 256;
    if (d->M <= 112) FAM_LAUNCH((partial_stream_kernel<7, 8>), grid, dim3(512), 0, s, pa, kper);
    else if (d->M <= 128) FAM_LAUNCH((partial_stream_kernel<8, 8>), grid, dim3(512), 0, s, pa, kper);
    else FAM_LAUNCH((partial_stream_kernel<9, 8>), grid, dim3(512), 0, s, pa, kper);
    return fam_host::check_launch("fam_gemm");
  }
  // (a normalising prologue over K > 1024 would not fit the 16-wave skinny variant's
  // registers; the folded LayerNorm runs K in chunks on 8 waves)
  const bool skinny = d->M <= 64 && (d->prologue == FAM_PRO_NONE || d->prologue == FAM_PRO_LN_FOLDED || d->K <= 1024);
  if (skinny && d->M <= 16) launch_skinny_k<1>(a, d->prologue, s);
  else if (skinny && d->M <= 32) launch_skinny_k<2>(a, d->prologue, s);
  else if (skinny) launch_skinny_k<4>(a, d->prologue, s);
  else if (big_ok(d)) {
    int fm = 8, fn = 8;
    big_plan(d->M, d->N, d->act, &fm, &fn, true);
    if (fm == 8) launch_big<8, 8>(a, s);
    else if (fm == 7) launch_big<7, 8>(a, s);
    else if (fm == 4 && fn == 3) launch_big<4, 3>(a, s);
    else if (fm == 4 && !big_prefers_64(d->M, d->N, d->K)) {
      // at most one 128 x 128 workgroup per CU: two K groups per workgroup (an even block count)
      const int64_t tiles = ((d->M + 127) / 128) * ((d->N + 127) / 128);
      if (tiles <= fam_host::device_cus() && (d->K / 64) % 2 == 0) launch_big<4, 4, 2>(a, s);
      else launch_big<4, 4>(a, s);
    } else launch_big<2, 2>(a, s);
  } else if (round_up(d->M, 128) / 128 * (round_up(d->N, 128) / 128) >= 200) launch_tiled<128, 128, 2>(a, d->prologue, s);
  else launch_tiled<64, 64, 2>(a, d->prologue, s);
  return fam_host::check_launch("fam_gemm");
}


// fam_gemm with a workspace: products inside the big kernel's envelope may split K over
// workgroups (big_plan_split), the fp32 planes summed in split order by fam_rowop, which also
// applies the bias / activation / gate / residual epilogue; everything else is fam_gemm.
extern "C" int64_t fam_gemm_ws_floats(int64_t M, int64_t N, int64_t K) {
  if (M < 128 || N < 1 || N % 4 != 0 || K < 128 || K % 64) return 0;
  // the planes of the split the unconstrained plan picks (deterministic for the device)
  int fm = 8, fn = 8, ks = 1;
  big_plan_split(M, N, K, INT64_MAX, false, &fm, &fn, &ks);
  return ks > 1 ? (int64_t)ks * M * N : 0;
}

extern "C" int fam_gemm_ws(const fam_gemm_desc* d, float* ws, int64_t ws_floats, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_gemm_ws: null descriptor");
  FAM_REQUIRE(ws_floats >= 0 && (ws_floats == 0 || (ws && ((uintptr_t)ws & 15u) == 0)), FAM_ERR_INVALID_ARG,
              "fam_gemm_ws: workspace must be 16-byte aligned");
  if (!big_ok(d) || d->M < 128 || ws_floats < 2 * d->M * d->N || d->N % 4 != 0 || d->act > FAM_ACT_GELU_ERF)
    return fam_gemm(d, stream);
  int fm = 8, fn = 8, ks = 1;
  big_plan_split(d->M, d->N, d->K, ws_floats, false, &fm, &fn, &ks);
  if (ks == 1) return fam_gemm(d, stream);
  GemmArgs a{};
  a.a = (const bf16*)d->a; a.lda = d->lda;
  a.w = (const bf16*)d->w; a.ldw = d->ldw;
  a.out = (bf16*)ws; a.ldo = d->N; a.out_f32 = 1;
  a.M = d->M; a.N = d->N; a.K = d->K; a.rpb = d->M;
  hipStream_t s = (hipStream_t)stream;
  if (fm == 8) launch_big<8, 8>(a, s, ks);
  else if (fm == 7) launch_big<7, 8>(a, s, ks);
  else if (fm == 4) launch_big<4, 4>(a, s, ks);
  else launch_big<2, 2>(a, s, ks);
  const int rc = fam_host::check_launch("fam_gemm_ws");
  if (rc != FAM_OK) return rc;
  fam_rowop_desc r{};
  r.src = FAM_ROWSRC_PARTIALS;
  r.partials = ws; r.splits = ks; r.split_stride = d->M * d->N; r.ldp = d->N;
  r.M = d->M; r.N = d->N;
  r.bias = d->bias; r.act = d->act;
  r.res = d->res; r.ldr = d->ldr;
  r.gate = d->gate; r.gate_bs = d->gate_bs; r.gate_rs = d->gate_rs; r.gate_ns = d->gate_ns;
  r.rows_per_batch = d->rows_per_batch;
  r.out = d->out; r.ldo = d->ldo; r.out_f32 = d->out_f32;
  r.norm = FAM_ROWNORM_NONE;
  return fam_rowop(&r, stream);
}


// Split plan of fam_gemm_partial.  Above 64 rows, first the streaming kernel: 128 columns per
// workgroup (64 when that is what gives every split 3 chunks), as many K splits as one round
// over the CUs allows, each split a whole number of 256-wide chunks; it runs when every
// workgroup gets at least 3 chunks to pipeline (steps returns -chunks, *nwv the waves).  Otherwise the wide kernel (one 512-wide K slice per workgroup, steps 0)
// when it alone fills the chip.  Otherwise, and up to 64 rows always, STEPS (32-wide k-steps
// per wave; a workgroup covers 4*32*STEPS of K) is the longest of 8, 4, 2, 1 that still gives
// >= 256 workgroups (one per CU), so the partial planes are as few as the machine's width
// allows; above 64 rows the eight m-tiles' activation fragments cap STEPS at 4 (registers).
static void partial_plan(int64_t M, int64_t N, int64_t K, int* steps, int* splits, int* nwv = nullptr) {
  const int64_t groups = (N + 15) / 16;
  const int64_t ksteps = (K + 31) / 32;
  if (M > 64) {
    const int64_t chunks = (K + 255) / 256;
    for (int w : {8, 4}) {
      if (w == 4 && M > 128) break;   // 9 m-tiles only with 8 waves
      const int64_t nblk = (N + 16 * w - 1) / (16 * w);
      const int64_t smax = std::max((int64_t)1, (int64_t)fam_host::device_cus() / nblk);
      const int64_t c = (chunks + std::min(chunks, smax) - 1) / std::min(chunks, smax);
      if (c >= 3) {
        *steps = -(int)c;
        *splits = (int)((chunks + c - 1) / c);
        if (nwv) *nwv = w;
        return;
      }
    }
  }
  if (M > 64 && ((N + 127) / 128) * ((K + 511) / 512) >= 128) {
    *steps = 0;
    *splits = (int)((K + 511) / 512);
    return;
  }
  int st = M > 64 ? 4 : 8;
  while (st > 1 && ((ksteps + 4 * st - 1) / (4 * st)) * groups < 256) st >>= 1;
  *steps = st;
  *splits = (int)((ksteps + 4 * st - 1) / (4 * st));
  if (M <= 64) {
    // two 16-column strips per workgroup sharing one LDS-staged 512-wide activation slice
    // halve the activation re-reads of the register kernel's one-strip workgroups; measured
    // faster at M = 32 once that still fills >= 192 workgroups (9216 x 1024: 10.5 -> 6.8 us;
    // 1024 x 3072: 5.1 -> 4.3 us), taken unless it multiplies the partial planes the row
    // kernel sums by more than 1.5
    const int64_t wsp = (K + 511) / 512, wblk = (N + 31) / 32;
    if (wblk * wsp >= 192 && wsp <= std::max((int64_t)2, (int64_t)(*splits) * 3 / 2)) {
      *steps = 0;
      *splits = (int)wsp;
    }
  }
}

// Above 128 rows (<= 144) only the streaming plan runs; 0 when it does not apply.
// above 144 rows: the big kernel writes the planes (K a multiple of 64, at least 128; N % 4 == 0)
static bool partial_big_shape(int64_t M, int64_t N, int64_t K) {
  return M > 144 && N >= 4 && N % 4 == 0 && K >= 128 && K % 64 == 0;
}

extern "C" int fam_gemm_partial_splits(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (M > 144) {
    if (!partial_big_shape(M, N, K)) return 0;
    int fm = 8, fn = 8, ks = 1;
    big_plan_split(M, N, K, INT64_MAX, true, &fm, &fn, &ks);
    return ks;
  }
  int st, sp;
  partial_plan(M, N, K, &st, &sp);
  return M > 128 && st >= 0 ? 0 : sp;
}

template <int MT>
static void launch_partial(const PartArgs& a, int steps, int splits, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 15) / 16), (unsigned)splits);
  switch (steps) {
    case 1: FAM_LAUNCH((partial_kernel<MT, 1>), grid, dim3(256), 0, s, a); break;
    case 2: FAM_LAUNCH((partial_kernel<MT, 2>), grid, dim3(256), 0, s, a); break;
    case 4: FAM_LAUNCH((partial_kernel<MT, 4>), grid, dim3(256), 0, s, a); break;
    default:
      if constexpr (MT <= 4) FAM_LAUNCH((partial_kernel<MT, 8>), grid, dim3(256), 0, s, a);
      break;
  }
}

// Waves per workgroup of the wide kernel (one 16-column strip each): the workgroup holds the
// 135 KB activation slice in LDS, so one runs per CU; the estimate is rounds over the CUs
// times the bytes a workgroup loads (weights 16 NWV x 512, activations M x 512).
static void launch_partial_wide(const PartArgs& a, int splits, hipStream_t s) {
  if (a.M <= 64) {   // two strips per workgroup (partial_plan)
    const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)splits);
    if (a.M <= 16) FAM_LAUNCH((partial_wide_kernel<1, 2>), grid, dim3(128), 0, s, a);
    else if (a.M <= 32) FAM_LAUNCH((partial_wide_kernel<2, 2>), grid, dim3(128), 0, s, a);
    else FAM_LAUNCH((partial_wide_kernel<4, 2>), grid, dim3(128), 0, s, a);
    return;
  }
  const int64_t cus = fam_host::device_cus();
  int best = 4;
  int64_t best_cost = -1;
  for (int nwv : {4, 6, 8}) {
    const int64_t wgs = (a.N + 16 * nwv - 1) / (16 * nwv) * splits;
    const int64_t cost = (wgs + cus - 1) / cus * (16 * nwv + a.M);
    if (best_cost < 0 || cost < best_cost) { best_cost = cost; best = nwv; }
  }
  const unsigned gy = (unsigned)splits;
  if (best == 8) FAM_LAUNCH((partial_wide_kernel<8, 8>), dim3((unsigned)((a.N + 127) / 128), gy), dim3(512), 0, s, a);
  else if (best == 6) FAM_LAUNCH((partial_wide_kernel<8, 6>), dim3((unsigned)((a.N + 95) / 96), gy), dim3(384), 0, s, a);
  else FAM_LAUNCH((partial_wide_kernel<8, 4>), dim3((unsigned)((a.N + 63) / 64), gy), dim3(256), 0, s, a);
}

extern "C" int fam_gemm_partial(const void* a, int64_t lda, const void* w, int64_t ldw, float* partials,
                                int64_t M, int64_t N, int64_t K, void* stream) {
  FAM_REQUIRE(a && w && partials, FAM_ERR_INVALID_ARG, "fam_gemm_partial: null pointer");
  FAM_REQUIRE(M >= 0 && N >= 1 && K >= 8 && K % 8 == 0, FAM_ERR_INVALID_ARG,
              "fam_gemm_partial: need M >= 0, N >= 1, K a positive multiple of 8 (M=%lld N=%lld K=%lld)",
              (long long)M, (long long)N, (long long)K);
  if (M > 144) {
    // the big kernel's split-K planes (raw fp32; one plane is its fp32 output without epilogue)
    FAM_REQUIRE(partial_big_shape(M, N, K), FAM_ERR_UNSUPPORTED,
                "fam_gemm_partial: above 144 rows N must be a multiple of 4 and K a multiple of 64, >= 128 "
                "(fam_gemm_partial_splits returns 0 otherwise; M=%lld N=%lld K=%lld)",
                (long long)M, (long long)N, (long long)K);
    FAM_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0 && fam_host::aligned16(a) &&
                    fam_host::aligned16(w) && fam_host::aligned16(partials),
                FAM_ERR_INVALID_ARG, "fam_gemm_partial: lda/ldw >= K and multiples of 8, 16-byte aligned pointers");
    FAM_REQUIRE((M + 256) * lda * 2 < (1LL << 31) && (N + 256) * ldw * 2 < (1LL << 31), FAM_ERR_UNSUPPORTED,
                "fam_gemm_partial: above 144 rows (M + 256) * lda * 2 and (N + 256) * ldw * 2 must be < 2^31 bytes");
    int fm = 8, fn = 8, ks = 1;
    big_plan_split(M, N, K, INT64_MAX, true, &fm, &fn, &ks);
    GemmArgs g{};
    g.a = (const bf16*)a; g.lda = lda;
    g.w = (const bf16*)w; g.ldw = ldw;
    g.out = (bf16*)partials; g.ldo = N; g.out_f32 = 1;
    g.M = M; g.N = N; g.K = K; g.rpb = M;
    hipStream_t s = (hipStream_t)stream;
    if (fm == 8) launch_big<8, 8>(g, s, ks, true);
    else if (fm == 7) launch_big<7, 8>(g, s, ks, true);
    else if (fm == 4) launch_big<4, 4>(g, s, ks, true);
    else launch_big<2, 2>(g, s, ks, true);
    return fam_host::check_launch("fam_gemm_partial");
  }
  FAM_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0, FAM_ERR_INVALID_ARG,
              "fam_gemm_partial: lda/ldw must be >= K and multiples of 8");
  FAM_REQUIRE(fam_host::aligned16(a) && fam_host::aligned16(w) && fam_host::aligned16(partials), FAM_ERR_INVALID_ARG,
              "fam_gemm_partial: a, w and partials must be 16-byte aligned");
  FAM_REQUIRE((N + 15) / 16 <= 2147483647LL, FAM_ERR_UNSUPPORTED, "fam_gemm_partial: N too large");
  // above 64 rows the streaming kernel addresses the activations and a workgroup's <= 128 weight
  // rows through 32-bit buffer descriptors whose out-of-range offset is 2^31: both spans must
  // stay below it
  FAM_REQUIRE(M <= 64 || (M * lda * 2 < (1LL << 31) && ldw < (1LL << 23) && N < (1LL << 31)), FAM_ERR_UNSUPPORTED,
              "fam_gemm_partial: above 64 rows M * lda * 2 must be < 2^31 bytes and ldw < 2^23 elements "
              "(M=%lld lda=%lld ldw=%lld)", (long long)M, (long long)lda, (long long)ldw);
  if (M == 0) return FAM_OK;
  int steps, splits, nwv = 8;
  partial_plan(M, N, K, &steps, &splits, &nwv);
  FAM_REQUIRE(M <= 128 || steps < 0, FAM_ERR_UNSUPPORTED,
              "fam_gemm_partial: above 128 rows only the streaming plan runs (>= 3 chunks of 256 per split with "
              "128-column workgroups; fam_gemm_partial_splits returns 0 otherwise)");
  PartArgs pa{(const bf16*)a, lda, (const bf16*)w, ldw, partials, M, N, K};
  hipStream_t s = (hipStream_t)stream;
  if (steps < 0) {
    const dim3 grid((unsigned)((N + 16 * nwv - 1) / (16 * nwv)), (unsigned)splits);
    const int kper = -steps * 256;
    if (nwv == 8) {
      if (M <= 112) FAM_LAUNCH((partial_stream_kernel<7, 8>), grid, dim3(512), 0, s, pa, kper);
      else if (M <= 128) FAM_LAUNCH((partial_stream_kernel<8, 8>), grid, dim3(512), 0, s, pa, kper);
      else FAM_LAUNCH((partial_stream_kernel<9, 8>), grid, dim3(512), 0, s, pa, kper);
    } else {
      if (M <= 112) FAM_LAUNCH((partial_stream_kernel<7, 4>), grid, dim3(256), 0, s, pa, kper);
      else FAM_LAUNCH((partial_stream_kernel<8, 4>), grid, dim3(256), 0, s, pa, kper);
    }
  } else if (steps == 0) launch_partial_wide(pa, splits, s);
  else if (M <= 16) launch_partial<1>(pa, steps, splits, s);
  else if (M <= 32) launch_partial<2>(pa, steps, splits, s);
  else if (M <= 64) launch_partial<4>(pa, steps, splits, s);
  else launch_partial<8>(pa, steps, splits, s);
  return fam_host::check_launch("fam_gemm_partial");
}

template <int MT, int NW>
static void launch_final_steps(const FinalArgs& a, int steps, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 15) / 16));
  switch (steps) {
    case 1: FAM_LAUNCH((final_kernel<MT, NW, 1>), grid, dim3(NW * 64), 0, s, a); break;
    case 2: FAM_LAUNCH((final_kernel<MT, NW, 2>), grid, dim3(NW * 64), 0, s, a); break;
    case 4: FAM_LAUNCH((final_kernel<MT, NW, 4>), grid, dim3(NW * 64), 0, s, a); break;
    default: FAM_LAUNCH((final_kernel<MT, NW, 8>), grid, dim3(NW * 64), 0, s, a); break;
  }
}

template <int MT>
static void launch_final(const FinalArgs& a, hipStream_t s) {
  // K <= 1024: 4 waves; longer: 16 waves; k-steps per wave 1, 2, 4 or 8.  Graph-timed at
  // M = 32, K = 1024 (N = 1024 / 3072 / 4096), 4 waves of 8 k-steps beat 8 waves of 4 by
  // 0.1-0.3 us a launch (the 4-way merge of the wave sums is shorter); above K = 1024 the 16
  // waves keep each wave's loads at 8 k-steps
  const int64_t ksteps = (a.K + 31) / 32;
  const int nw = ksteps <= 32 ? 4 : 16;
  int steps = 1;
  while (steps * nw < ksteps) steps <<= 1;
  if (nw == 4) launch_final_steps<MT, 4>(a, steps, s);
  else launch_final_steps<MT, 16>(a, steps, s);
}

extern "C" int fam_gemm_final(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, int act,
                              void* out, int64_t ldo, float* sumsq, int64_t M, int64_t N, int64_t K, void* stream) {
  FAM_REQUIRE(a && w && out, FAM_ERR_INVALID_ARG, "fam_gemm_final: a, w and out must be non-null");
  FAM_REQUIRE(M >= 0 && M <= 64 && N >= 1 && K >= 8 && K % 8 == 0 && K <= 4096, FAM_ERR_INVALID_ARG,
              "fam_gemm_final: need 0 <= M <= 64, N >= 1, K a multiple of 8 in [8, 4096] (M=%lld N=%lld K=%lld)",
              (long long)M, (long long)N, (long long)K);
  FAM_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0 && ldo >= N, FAM_ERR_INVALID_ARG,
              "fam_gemm_final: lda/ldw must be >= K and multiples of 8, ldo >= N");
  FAM_REQUIRE(fam_host::aligned16(a) && fam_host::aligned16(w) && (reinterpret_cast<uintptr_t>(out) & 7u) == 0,
              FAM_ERR_INVALID_ARG, "fam_gemm_final: a, w 16-byte and out 8-byte aligned");
  FAM_REQUIRE(act >= FAM_ACT_NONE && act <= FAM_ACT_GELU_ERF, FAM_ERR_INVALID_ARG, "fam_gemm_final: unknown act %d", act);
  FAM_REQUIRE((N + 15) / 16 <= 2147483647LL, FAM_ERR_UNSUPPORTED, "fam_gemm_final: N too large");
  if (M == 0) return FAM_OK;
  FinalArgs fa{(const bf16*)a, lda, (const bf16*)w, ldw, (const bf16*)bias, act, (bf16*)out, ldo, sumsq, M, N, K};
  hipStream_t s = (hipStream_t)stream;
  if (M <= 16) launch_final<1>(fa, s);
  else if (M <= 32) launch_final<2>(fa, s);
  else launch_final<4>(fa, s);
  return fam_host::check_launch("fam_gemm_final");
}
