// The denoise loop of a tiny-hidden action expert (hidden 32) in two launches per block step.
//
// Experts such as the CAE-FastWAM action expert (hidden 32, 24 x 128 attention, 30 blocks,
// 8 action tokens over 98 cached video tokens) or the compact expert of config 3 (hidden 32,
// 4 x 8 heads) move almost no data per block step: the [S, 32] residual rows are 1 KB, the
// block's weights a few hundred KB.  The generic plan (a projection kernel plus a row kernel per
// linear layer) is then a chain of ~12 dependent launches per block step, each mostly launch
// latency.  Here every block step is two phases, each one launch:
//
//   self  (g, b): finish the previous block on the 32-wide rows (x += cross o + bias, then the
//                 FFN with its AdaLN and gate; at the first block of a step also the head, the
//                 Euler update of the chunk and the action encoder), AdaLN1, q/k/v of the heads
//                 in column slice g, RMSNorm + 1-D RoPE, attention over [video K/V ; action
//                 K/V], and the slice's share of the o projection (fp32 partial);
//   cross (g, b): x += gate_msa (sum of the o partials + bias), affine LayerNorm3, the slice's
//                 cross-attention query + RMSNorm, attention over the context, and the slice's
//                 share of the cross o projection.  A slice wider than the 32-wide rows attends
//                 in the space of the context rows (attend_ctx) instead of reading its K / V.
//
// The phase boundaries are exactly the two cross-head reductions of a block (the o projections
// sum over all heads); everything else a workgroup needs it recomputes from the previous
// phase's partials, in a fixed order, so every workgroup of a batch row holds bit-identical
// rows and slice 0 alone stores them.  With a single 32-wide slice and few batch rows (config
// 3's compact expert over 1560 context keys) the cross phase also splits the context over KS
// workgroups: each stores its split's unnormalised output with the running max and sum, and
// the next phase merges the splits in split order and applies the (32 x 32) cross o projection
// itself, where the other layouts read the o partials.  The RMSNorm of q / k / cross q runs over all A columns:
// a workgroup that sees only its slice gets the row's sum of squares from the layer's Gram
// matrix G = W^T W (hi + lo bf16 parts, two MFMAs), sum_j q_j^2 = h G h + 2 h.(W^T b) + |b|^2,
// since the input row h is only 32 wide.
//
// Products run on v_mfma_f32_16x16x32_bf16 in the transposed form D^T = W X^T (weight rows as
// the A operand from global memory, the <= 16 token rows as the B operand from LDS); attention
// uses the transposed scores S^T = K Q^T with a block-diagonal Q^T so that several small heads
// of a slice share one MFMA (column (head, token)), and O^T = V^T P^T from a wave-private V tile
// read back by transposing LDS reads.  Every global load a phase needs that does not depend on
// the rows (weights, the first video / context block) is issued before the first barrier, and
// the barriers wait for LDS traffic only (lds_barrier): a global store is read by the next
// launch, never by this one, so no barrier has to drain the loads still in flight.
#include <algorithm>

#include "fam_common.h"

namespace fam {

constexpr int TH = 32;    // hidden width
constexpr int TS = 16;    // action tokens per chunk (one MFMA column block)
constexpr int TF = 256;   // FFN width
constexpr int TDA = 32;   // action dim
constexpr int TG = 64;    // column slices (G)

namespace {

struct TinyArgs {
  int B, S, A, DH, F, Da, L, T, Sv, Lc, G;
  float eps, scale_log2;
  const bf16* noise;
  const bf16* mods;
  const bf16* deltas;
  const float* rcos;
  const float* rsin;
  const bf16* ctxkv;
  int64_t ctx_ld;
  const bf16* const* vk;
  const bf16* const* vv;
  int64_t v_bs, v_rs;
  const uint8_t* mask;
  int64_t mask_rs;
  const bf16 *enc_w, *enc_b, *head_w, *head_b;
  const bf16 *qkv_w, *qkv_b, *nq_w, *nk_w, *o_w, *o_b, *n3_w, *n3_b, *cq_w, *cq_b, *cnq_w, *co_w, *co_b, *ff0_w, *ff0_b,
      *ff2_w, *ff2_b;
  const bf16* gram;
  const float* gram_c;
  const float* gram_b;
  float *lat, *xa, *xb, *part_s, *part_c, *out;
  const bf16* ctx_emb;
  int64_t ctx_emb_ld;
  const bf16 *ck_wt, *ck_b, *cnk_w, *cv_w, *cv_b;
  float* ctx_rs;
  int Lcp;   // keys of ctx_rs per layer (Lc rounded up to 32)
  int KS;    // context splits of the cross phase (1: none)
  float* part_x;   // KS > 1: [B][KS][32 columns][W + 4]: o (unnormalised), max, sum
  int p0, p1;
};

template <int W, int NCB>
struct TinySmem {
  float x[TS][TH + 4];               // residual rows (fp32)
  float lat[TS][TDA];                // the chunk (fp32)
  bf16 ew[TH * TDA];                 // encoder weight [32, Da]
  bf16 hw[TDA * TH];                 // head weight [Da, 32]
  __attribute__((aligned(16))) bf16 hb[TS][TH + 8];   // normalised rows: B operand of the next product
  float ss[3][TS];                   // row sums of squares (q, k | cross q)
  __attribute__((aligned(16))) bf16 q[TS][W + 8];
  __attribute__((aligned(16))) bf16 k[TS][W + 8];
  __attribute__((aligned(16))) bf16 v[TS][W + 8];
  __attribute__((aligned(16))) bf16 o[TS][W + 8];
  __attribute__((aligned(16))) bf16 vt[4][32][W + 16];   // wave-private V tiles
  union U {
    float raw[TS][3 * W + 4];                            // q | k | v before the norm (fp32)
    struct {
      __attribute__((aligned(16))) bf16 hid[TS][TF + 8];  // FFN hidden rows
      float red[4][TS][TH + 4];                          // per-wave FFN-down partials
    } f;
    struct {
      float m[4][NCB * 16], l[4][NCB * 16];
      float acc[4][NCB * 16][W + 8];                     // [wave][column][dim]: W + 8 keeps 16-byte
    } mg;                                                // accesses of 32 lanes in distinct banks
  } u;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf(const bf16* p) { return to_f(*p); }

// ---------------------------------------------------------------------------------------
// Row ops on the [S, 32] rows: 16 threads per row, 2 elements each (tid = 16 s + j).
struct RowMod {   // per-thread modulation / affine pairs of a row op, loaded early
  bf16x2 a, c;    // AdaLN: shift, scale; affine LN: weight, bias
};

__device__ __forceinline__ RowMod row_mod_load(const bf16* pa, const bf16* pc) {
  const int j = threadIdx.x & 15;
  RowMod m;
  m.a = *reinterpret_cast<const bf16x2*>(pa + 2 * j);
  m.c = *reinterpret_cast<const bf16x2*>(pc + 2 * j);
  return m;
}

// hb[s] = bf16(LN(x[s]) (1 + scale) + shift)  (adaln)  or  bf16(LN(x[s]) w + b)  (affine);
// rows s >= S are zero.
template <int W, int NCB>
__device__ __forceinline__ void row_norm(TinySmem<W, NCB>& sm, int S, float eps, RowMod m, bool adaln) {
  const int s = threadIdx.x >> 4, j = threadIdx.x & 15;
  const float x0 = sm.x[s][2 * j], x1 = sm.x[s][2 * j + 1];
  float sum = x0 + x1;
  sum = row16_sum(sum);
  const float mean = sum * (1.0f / TH);
  const float d0 = x0 - mean, d1 = x1 - mean;
  float var = d0 * d0 + d1 * d1;
  var = row16_sum(var);
  const float rstd = rsqrtf(var * (1.0f / TH) + eps);
  float y0 = d0 * rstd, y1 = d1 * rstd;
  if (adaln) {
    y0 = y0 * (1.0f + to_f(m.c[0])) + to_f(m.a[0]);
    y1 = y1 * (1.0f + to_f(m.c[1])) + to_f(m.a[1]);
  } else {
    y0 = y0 * to_f(m.a[0]) + to_f(m.c[0]);
    y1 = y1 * to_f(m.a[1]) + to_f(m.c[1]);
  }
  if (s >= S) y0 = y1 = 0.f;
  bf16x2 h;
  h[0] = to_bf(y0);
  h[1] = to_bf(y1);
  *reinterpret_cast<bf16x2*>(&sm.hb[s][2 * j]) = h;
}

// B operand (X^T, k-block 0 of the 32-wide rows) of a lane: row l16, columns 8 lg .. 8 lg + 7
template <int W, int NCB>
__device__ __forceinline__ bf16x8 hb_frag(TinySmem<W, NCB>& sm) {
  const int lane = threadIdx.x & 63;
  return *reinterpret_cast<const bf16x8*>(&sm.hb[lane & 15][8 * (lane >> 4)]);
}

// ---------------------------------------------------------------------------------------
// FFN of block lp: x += gate (W2 GELU(W1 AdaLN(x) + b1) + b2), the weights' fragments
// prefetched by ffn_load.  F/16 up tiles over the 4 waves; F/32 down k-blocks over the waves,
// their partials summed in wave order.
struct FfnFrags {
  bf16x8 up[TF / 64];
  bf16x4 ub[TF / 64];
  bf16x8 dn[TF / 128][2];
};

__device__ __forceinline__ void ffn_load(const TinyArgs& a, int lp, FfnFrags& f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  const int F = a.F, NU = F / 16, ND = F / 32;
  const bf16* w1 = a.ff0_w + (size_t)lp * F * TH;
  const bf16* b1 = a.ff0_b + (size_t)lp * F;
  const bf16* w2 = a.ff2_w + (size_t)lp * TH * F;
#pragma unroll
  for (int i = 0; i < TF / 64; ++i) {
    int tau = wave + 4 * i;
    tau = tau < NU ? tau : NU - 1;
    f.up[i] = load8(w1 + (size_t)(tau * 16 + l16) * TH + lg * 8);
    f.ub[i] = *reinterpret_cast<const bf16x4*>(b1 + tau * 16 + lg * 4);
  }
#pragma unroll
  for (int j = 0; j < TF / 128; ++j) {
    int kb = wave + 4 * j;
    kb = kb < ND ? kb : ND - 1;
#pragma unroll
    for (int t = 0; t < 2; ++t) f.dn[j][t] = load8(w2 + (size_t)(t * 16 + l16) * F + kb * 32 + lg * 8);
  }
}

// x += gate * (ffn(hb) + b2); hb holds AdaLN(x) already; ends with a barrier.
template <int W, int NCB>
__device__ __forceinline__ void ffn_apply(const TinyArgs& a, TinySmem<W, NCB>& sm, const FfnFrags& f, bf16x2 b2,
                                          bf16x2 gate) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  const int F = a.F, NU = F / 16, ND = F / 32;
  const bf16x8 hf = hb_frag(sm);
#pragma unroll
  for (int i = 0; i < TF / 64; ++i) {
    const int tau = wave + 4 * i;
    if (tau < NU) {
      const f32x4 d = mfma16(f.up[i], hf, f32x4{0.f, 0.f, 0.f, 0.f});   // D[n = 16 tau + 4 lg + e][s = l16]
      bf16x4 hv;
#pragma unroll
      for (int e = 0; e < 4; ++e) hv[e] = to_bf(gelu_tanh(d[e] + to_f(f.ub[i][e])));
      *reinterpret_cast<bf16x4*>(&sm.u.f.hid[l16][tau * 16 + lg * 4]) = hv;
    }
  }
  lds_barrier();
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int j = 0; j < TF / 128; ++j) {
    const int kb = wave + 4 * j;
    if (kb < ND) {
      const bf16x8 bfr = *reinterpret_cast<const bf16x8*>(&sm.u.f.hid[l16][kb * 32 + lg * 8]);
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[t] = mfma16(f.dn[j][t], bfr, acc[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) sm.u.f.red[wave][l16][t * 16 + lg * 4 + e] = acc[t][e];
  lds_barrier();
  const int s = threadIdx.x >> 4, j = threadIdx.x & 15;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 2 * j + c;
    const float y = ((sm.u.f.red[0][s][n] + sm.u.f.red[1][s][n]) + (sm.u.f.red[2][s][n] + sm.u.f.red[3][s][n])) +
                    to_f(b2[c]);
    sm.x[s][n] += to_f(gate[c]) * y;
  }
  lds_barrier();
}

// ---------------------------------------------------------------------------------------
// Column-slice products of the [S, 32] rows: D^T[n][s] = sum_k W[n][k] hb[s][k] over 16-row
// tiles of W (K = 32, one MFMA per tile).
template <int W>
struct SliceFrags {
  static constexpr int NT = 3 * W / 16;        // q, k, v tiles of the slice
  static constexpr int PW = (NT + 3) / 4;      // tiles per wave
  bf16x8 w[PW];
  bf16x4 b[PW];
};

// Gram fragments of one weight (hi, lo parts of two 16-row tiles) and W^T b
struct GramFrags {
  bf16x8 g[2][2];
  f32x4 c[2];
  float beta;
};

__device__ __forceinline__ void gram_load(const TinyArgs& a, int l, int which, GramFrags& gf) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
      gf.g[t][hl] = load8(a.gram + ((size_t)((l * 4 + which) * 2 + hl) * TH + t * 16 + l16) * TH + lg * 8);
    gf.c[t] = *reinterpret_cast<const f32x4*>(a.gram_c + (size_t)(l * 4 + which) * TH + t * 16 + lg * 4);
  }
  gf.beta = a.gram_b[l * 4 + which];
}

// sum_j q_j^2 of row l16 from the Gram form; lanes of group 0 store it (rows < S)
template <int W, int NCB>
__device__ __forceinline__ void gram_sumsq(TinySmem<W, NCB>& sm, const GramFrags& gf, int which, int S) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
  const bf16x8 hf = hb_frag(sm);
  float part = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x4 d = mfma16(gf.g[t][0], hf, f32x4{0.f, 0.f, 0.f, 0.f});
    d = mfma16(gf.g[t][1], hf, d);   // (G h)[i = 16 t + 4 lg + e] of row l16
    const bf16x4 h4 = *reinterpret_cast<const bf16x4*>(&sm.hb[l16][t * 16 + lg * 4]);
#pragma unroll
    for (int e = 0; e < 4; ++e) part += to_f(h4[e]) * (d[e] + 2.0f * gf.c[t][e]);
  }
  part = group4_sum(part) + gf.beta;
  if (lg == 0 && l16 < S) sm.ss[which][l16] = part;
}

// ---------------------------------------------------------------------------------------
// Attention of the slice's heads: S queries (columns (head, token) of a block-diagonal Q^T)
// over keys [segment 0 (global rows) ; segment 1 (the action rows in LDS)], 32-key blocks
// round-robin over the 4 waves, online softmax per column, waves merged in order -> sm.o.
// Keys past the end load a valid row of the same operand (row 0), never zero-selected right
// after the load: a select on a loaded value makes the compiler wait for that load before
// issuing the next one.  Such keys cost nothing downstream: their scores are masked to -inf
// (p = 0) and their finite values times p = 0 add 0.
template <int W>
struct KvBlock {
  bf16x8 k[2][W / 32];
  bf16x8 v[W / 16];
};

struct KvSrc {
  const bf16* k0;   // segment 0: row kk at k0 + kk * rs0 (slice columns)
  const bf16* v0;
  int64_t rs0;
  int n0, n1;       // keys of segment 0 and 1 (segment 1 = sm.k / sm.v rows)
};

template <int W, int NCB>
__device__ __forceinline__ void kv_load(TinySmem<W, NCB>& sm, const KvSrc& src, int blk, KvBlock<W>& kv) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
  const int n = src.n0 + src.n1;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int kk = blk * 32 + sub * 16 + l16;
#pragma unroll
    for (int kb = 0; kb < W / 32; ++kb) {
      const int col = kb * 32 + lg * 8;
      const bf16* p = kk < src.n0 ? src.k0 + kk * src.rs0 + col : &sm.k[kk < n ? kk - src.n0 : 0][col];
      kv.k[sub][kb] = load8(p);
    }
  }
  constexpr int CPR = W / 8;   // 16-byte chunks per row
#pragma unroll
  for (int i = 0; i < W / 16; ++i) {
    const int ci = lane + 64 * i, row = ci / CPR, c8 = ci - row * CPR;
    const int kk = blk * 32 + row;
    const bf16* p = kk < src.n0 ? src.v0 + kk * src.rs0 + c8 * 8 : &sm.v[kk < n ? kk - src.n0 : 0][c8 * 8];
    kv.v[i] = load8(p);
  }
}

// global-only variant for a block wholly inside segment 0 (prefetch before the rows exist)
template <int W>
__device__ __forceinline__ void kv_load_global(const KvSrc& src, int blk, KvBlock<W>& kv) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    int kk = blk * 32 + sub * 16 + l16;
    kk = kk < src.n0 ? kk : 0;
#pragma unroll
    for (int kb = 0; kb < W / 32; ++kb) kv.k[sub][kb] = load8(src.k0 + kk * src.rs0 + kb * 32 + lg * 8);
  }
  constexpr int CPR = W / 8;
#pragma unroll
  for (int i = 0; i < W / 16; ++i) {
    const int ci = lane + 64 * i, row = ci / CPR, c8 = ci - row * CPR;
    int kk = blk * 32 + row;
    kk = kk < src.n0 ? kk : 0;
    kv.v[i] = load8(src.v0 + kk * src.rs0 + c8 * 8);
  }
}

// Keys [n0, n) of a block prefetched by kv_load_global (which read row 0 for them) come from the
// action rows in LDS once they exist.
template <int W, int NCB>
__device__ __forceinline__ void kv_patch(TinySmem<W, NCB>& sm, const KvSrc& src, int blk, KvBlock<W>& kv) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
  const int n = src.n0 + src.n1;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int kk = blk * 32 + sub * 16 + l16;
    const bool act = kk >= src.n0 && kk < n;
#pragma unroll
    for (int kb = 0; kb < W / 32; ++kb) {
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(&sm.k[act ? kk - src.n0 : 0][kb * 32 + lg * 8]);
      kv.k[sub][kb] = act ? x : kv.k[sub][kb];
    }
  }
  constexpr int CPR = W / 8;
#pragma unroll
  for (int i = 0; i < W / 16; ++i) {
    const int ci = lane + 64 * i, row = ci / CPR, c8 = ci - row * CPR;
    const int kk = blk * 32 + row;
    const bool act = kk >= src.n0 && kk < n;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(&sm.v[act ? kk - src.n0 : 0][c8 * 8]);
    kv.v[i] = act ? x : kv.v[i];
  }
}

// Online softmax of one 32-key block for one column block: sc[sub][e] is the score (exp2 units,
// -inf when masked) of key 16 sub + 4 lg + e of column l16.  The running max moves only when a
// score passes it by more than 2^8 (exp2 units), so p <= 2^8 in between (exact in fp32, bf16 keeps
// its relative precision) and the accumulators are rescaled only on the blocks where some column
// of the wave moved (the first, mostly): returns true with alpha then.  pf: the P^T fragment.
__device__ __forceinline__ bool softmax_block(const float (&sc)[2][4], float& m, float& lsum, bf16x8& pf,
                                              float& alpha) {
  float mb = -INFINITY;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int e = 0; e < 4; ++e) mb = fmaxf(mb, sc[sub][e]);
  mb = group4_max(mb);
  const bool up = mb > m + 8.0f;
  const float mn = up ? mb : m;
  const float ms = mn == -INFINITY ? 0.f : mn;
  float ps = 0.f;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __builtin_amdgcn_exp2f(sc[sub][e] - ms);
      ps += p;
      pf[sub * 4 + e] = to_bf(p);
    }
  ps = group4_sum(ps);
  if (__any(up)) {
    alpha = __builtin_amdgcn_exp2f(m - ms);   // unchanged max: 1; -inf: 0
    lsum = lsum * alpha + ps;
    m = mn;
    return true;
  }
  lsum += ps;
  m = mn;
  return false;
}

// One 32-key block of a wave: V rows into the wave's tile, scores, online softmax, O^T += V^T P^T.
template <int W, int NCB>
__device__ __forceinline__ void attend_block(const TinyArgs& a, const KvBlock<W>& kv, int blk, int n,
                                             const uint8_t* mask, int64_t mask_rs, const bf16x8 (&qf)[NCB][W / 32],
                                             const int (&qs)[NCB], float (&m)[NCB], float (&lsum)[NCB],
                                             f32x4 (&acc)[W / 16][NCB], bf16 (*vt)[W + 16]) {
  constexpr int WK = W / 32, WT = W / 16, CPR = W / 8;
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
  // the block's V rows into the wave's tile
#pragma unroll
  for (int i = 0; i < WT; ++i) {
    const int ci = lane + 64 * i, row = ci / CPR, c8 = ci - row * CPR;
    *reinterpret_cast<bf16x8*>(&vt[row][c8 * 8]) = kv.v[i];
  }
  // scores of the block: keys 32 blk + 16 sub + 4 lg + e, column cb * 16 + l16
  bf16x8 pf[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    float sc[2][4];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < WK; ++kb) d = mfma16(kv.k[sub][kb], qf[cb][kb], d);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = blk * 32 + sub * 16 + lg * 4 + e;
        bool ok = kk < n;
        if (mask != nullptr) ok = ok && (qs[cb] < 0 || mask[(int64_t)qs[cb] * mask_rs + kk] != 0);
        sc[sub][e] = ok ? d[e] * a.scale_log2 : -INFINITY;
      }
    }
    float alpha;
    if (softmax_block(sc, m[cb], lsum[cb], pf[cb], alpha)) {
#pragma unroll
      for (int dt = 0; dt < WT; ++dt) acc[dt][cb] *= alpha;
    }
  }
  // O^T += V^T P^T: V^T fragment rows = dims 16 dt + l16, k = keys {4 lg..+3, 16 + 4 lg..+3}
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
#pragma unroll
  for (int dt = 0; dt < WT; ++dt) {
    const int key = lg * 4 + (l16 >> 2), dim = dt * 16 + 4 * (l16 & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&vt[key][dim]);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&vt[key + 16][dim]);
    const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const bf16x8 vf = __builtin_bit_cast(bf16x8, v8);
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[dt][cb] = mfma16(vf, pf[cb], acc[dt][cb]);
  }
}

// PD blocks of a wave in flight: PD = 1 for any key source; PD = 2 or 3 only for keys wholly in
// segment 0 (src.n1 == 0), as a ring of PD + 1 named register blocks (the loop unrolled by
// PD + 1, so no slot is indexed at run time) whose loads are all issued, past the end too
// (kv_load_global reads row 0 there), so the wait before each block counts exactly the loads
// issued after it.
// xout != nullptr: the merged state of this workgroup's keys goes there unnormalised, per column
// c = (head, token): [c][d] = the waves' sum of exp2(m_w - m) o_w over the head's dims d,
// [c][W] = m, [c][W + 1] = the matching sum of p; nothing is written to sm.o.
template <int PD, int W, int NCB>
__device__ __forceinline__ void attend(const TinyArgs& a, TinySmem<W, NCB>& sm, const KvSrc& src, const uint8_t* mask,
                                       int64_t mask_rs, KvBlock<W>& kv, bool prefetched, float* xout = nullptr) {
  constexpr int WK = W / 32, WT = W / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  const int S = a.S, DH = a.DH;
  const int dsh = __builtin_ctz(DH), nc = (W >> dsh) * S;
  const int n = src.n0 + src.n1, nblk = (n + 31) / 32;
  // Q^T fragments: column c = (head hh, token s); dims of other heads read as zero
  bf16x8 qf[NCB][WK];
  int qs[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int c = cb * 16 + l16, hh = c / S, s = c - hh * S;
    qs[cb] = c < nc ? s : -1;
#pragma unroll
    for (int kb = 0; kb < WK; ++kb) {
      const int d0 = kb * 32 + lg * 8;
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(&sm.q[c < nc ? s : 0][d0]);
      qf[cb][kb] = (c < nc && (d0 >> dsh) == hh) ? x : zero8();
    }
  }
  float m[NCB], lsum[NCB];
  f32x4 acc[WT][NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    m[cb] = -INFINITY;
    lsum[cb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < WT; ++dt) acc[dt][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  bf16(*vt)[W + 16] = sm.vt[wave];
  if constexpr (PD == 1) {
    if (prefetched && src.n1 > 0 && wave * 32 + 32 > src.n0) kv_patch(sm, src, wave, kv);
    if (!prefetched && wave < nblk) {
      if (src.n1 == 0)
        kv_load_global<W>(src, wave, kv);
      else
        kv_load(sm, src, wave, kv);
    }
    for (int blk = wave; blk < nblk; blk += 4) {
      // the wave's next block in flight while this one is computed
      KvBlock<W> nx;
      if (blk + 4 < nblk) {
        if (src.n1 == 0)
          kv_load_global<W>(src, blk + 4, nx);
        else
          kv_load(sm, src, blk + 4, nx);
      }
      attend_block<W, NCB>(a, kv, blk, n, mask, mask_rs, qf, qs, m, lsum, acc, vt);
      if (blk + 4 < nblk) kv = nx;
    }
  } else {
    static_assert(PD == 2 || PD == 3, "ring depth");
    // slot j of step j is consumed; the block PD steps ahead goes into the slot of step j - 1
    KvBlock<W> r0, r1, r2, r3;
    if (prefetched)
      r0 = kv;
    else
      kv_load_global<W>(src, wave, r0);
    kv_load_global<W>(src, wave + 4, r1);
    if constexpr (PD == 3) kv_load_global<W>(src, wave + 8, r2);
#define FAM_TINY_STEP(J, CUR, NXT)                                                                        \
  {                                                                                                       \
    const int blk = base + 4 * (J);                                                                       \
    kv_load_global<W>(src, blk + 4 * PD, NXT);                                                            \
    if (blk < nblk) attend_block<W, NCB>(a, CUR, blk, n, mask, mask_rs, qf, qs, m, lsum, acc, vt);       \
  }
    for (int base = wave; base < nblk; base += 4 * (PD + 1)) {
      if constexpr (PD == 3) {
        FAM_TINY_STEP(0, r0, r3)
        FAM_TINY_STEP(1, r1, r0)
        FAM_TINY_STEP(2, r2, r1)
        FAM_TINY_STEP(3, r3, r2)
      } else {
        FAM_TINY_STEP(0, r0, r2)
        FAM_TINY_STEP(1, r1, r0)
        FAM_TINY_STEP(2, r2, r1)
      }
    }
#undef FAM_TINY_STEP
  }
  // merge the waves' states through LDS, in wave order
  if (lg == 0) {
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      sm.u.mg.m[wave][cb * 16 + l16] = m[cb];
      sm.u.mg.l[wave][cb * 16 + l16] = lsum[cb];
    }
  }
#pragma unroll
  for (int dt = 0; dt < WT; ++dt)
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
      *reinterpret_cast<f32x4*>(&sm.u.mg.acc[wave][cb * 16 + l16][dt * 16 + lg * 4]) = acc[dt][cb];
  lds_barrier();
  // one thread per (token, 8 dims of one head): the waves' weights once, then two 16-byte reads
  // per wave (head_dim is a power of two: W and a multiple of it are)
  if (threadIdx.x < S * (W / 8)) {
    const int idx = threadIdx.x, s = idx / (W / 8), d0 = (idx - s * (W / 8)) * 8, c = (d0 >> dsh) * S + s;
    float mw[4], mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = sm.u.mg.m[w][c];
      mx = fmaxf(mx, mw[w]);
    }
    const float ms = mx == -INFINITY ? 0.f : mx;
    float f[4], den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      f[w] = __builtin_amdgcn_exp2f(mw[w] - ms);
      den += f[w] * sm.u.mg.l[w][c];
    }
    f32x4 n0 = f32x4{0.f, 0.f, 0.f, 0.f}, n1 = n0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      n0 += f[w] * *reinterpret_cast<const f32x4*>(&sm.u.mg.acc[w][c][d0]);
      n1 += f[w] * *reinterpret_cast<const f32x4*>(&sm.u.mg.acc[w][c][d0 + 4]);
    }
    if (xout != nullptr) {
      float* p = xout + (size_t)c * (W + 4);
      *reinterpret_cast<f32x4*>(p + d0) = n0;
      *reinterpret_cast<f32x4*>(p + d0 + 4) = n1;
      if ((d0 & (DH - 1)) == 0) *reinterpret_cast<f32x2*>(p + W) = f32x2{mx, den};
    } else {
      const float inv = den > 0.f ? 1.f / den : 0.f;
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = to_bf(n0[e] * inv);
        o[4 + e] = to_bf(n1[e] * inv);
      }
      *reinterpret_cast<bf16x8*>(&sm.o[s][d0]) = o;
    }
  }
  lds_barrier();
}

// ---------------------------------------------------------------------------------------
// The context splits of the previous cross phase (KS > 1; one 32-wide slice): thread (token s,
// 8 dims d0) loads the KS splits' outputs of its column c = (head of d0, s) early; the merge
// (splits in order, weights exp2(m_k - max m)) writes o = bf16(sum / den) to sm.o, and the cross
// o projection of the slice fills sm.u.f.red[0] (the other red planes zero) where the other
// layouts sum their o partials.
constexpr int TKS = 8;   // at most 8 context splits

struct XSplit {
  f32x4 o[TKS][2];
  f32x2 ml[TKS];
};

template <int W>
__device__ __forceinline__ void xsplit_issue(const TinyArgs& a, int b, XSplit& x) {
  const int tid = threadIdx.x, S = a.S;
  const int dsh = __builtin_ctz(a.DH);
  const int t = tid < S * (W / 8) ? tid : 0, s = t / (W / 8), d0 = (t - s * (W / 8)) * 8, c = (d0 >> dsh) * S + s;
#pragma unroll
  for (int k = 0; k < TKS; ++k) {
    const int kk = k < a.KS ? k : 0;
    const float* p = a.part_x + ((size_t)(b * a.KS + kk) * 32 + c) * (W + 4);
    x.o[k][0] = *reinterpret_cast<const f32x4*>(p + d0);
    x.o[k][1] = *reinterpret_cast<const f32x4*>(p + d0 + 4);
    x.ml[k] = *reinterpret_cast<const f32x2*>(p + W);
  }
}

template <int W, int NCB>
__device__ __forceinline__ void xsplit_merge(const TinyArgs& a, TinySmem<W, NCB>& sm, const XSplit& x,
                                             const bf16x8 (&of)[W / 32]) {
  const int tid = threadIdx.x, S = a.S, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  if (tid < S * (W / 8)) {
    const int s = tid / (W / 8), d0 = (tid - s * (W / 8)) * 8;
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < TKS; ++k)
      if (k < a.KS) mx = fmaxf(mx, x.ml[k][0]);
    const float ms = mx == -INFINITY ? 0.f : mx;
    float den = 0.f;
    f32x4 n0 = f32x4{0.f, 0.f, 0.f, 0.f}, n1 = n0;
#pragma unroll
    for (int k = 0; k < TKS; ++k) {
      if (k < a.KS) {
        const float f = __builtin_amdgcn_exp2f(x.ml[k][0] - ms);
        den += f * x.ml[k][1];
        n0 += f * x.o[k][0];
        n1 += f * x.o[k][1];
      }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = to_bf(n0[e] * inv);
      o[4 + e] = to_bf(n1[e] * inv);
    }
    *reinterpret_cast<bf16x8*>(&sm.o[s][d0]) = o;
  }
  lds_barrier();
  // part[s][n] = sum_d o[s][d] Wo[n][d]: waves 0, 1 one 16-row tile of the 32 outputs each
  const int NGI = min(4, 256 / (S * 8));
  if (wave < 2) {
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < W / 32; ++kb)
      d = mfma16(of[kb], *reinterpret_cast<const bf16x8*>(&sm.o[l16][kb * 32 + lg * 8]), d);
    if (l16 < S) *reinterpret_cast<f32x4*>(&sm.u.f.red[0][l16][wave * 16 + lg * 4]) = d;
  } else {
    for (int i = tid - 128; i < (NGI - 1) * TS * TH; i += 128) {
      const int gi = 1 + i / (TS * TH), r = i % (TS * TH);
      sm.u.f.red[gi][r / TH][r % TH] = 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Context attention in the 32-wide space of the context rows (slices wider than the rows).  For
// the key k = r (W_k h + b_k) * w_k of a context row h (r: its RMS factor over all A columns, w_k:
// the key norm weight) and the query q_c of column c = (head, token), zero outside its head,
//   q_c . k = r (h . Q_c + beta_c),   Q_c = W_k^T (q_c * w_k),   beta_c = b_k . (q_c * w_k),
// and the output is  sum_key p (W_v h + b_v) / l = W_v Z_c + b_v  with  Z_c = sum_key p h / l.
// A 32-key block then reads 2 KB of rows and 128 B of factors (the slice's K and V would be
// 4 W bytes per key), and its products are 32 deep.  Q_c and Z_c enter their products as hi + lo
// bf16 parts; q_c * w_k is rounded to bf16 once (sm.q holds it).  The block's 32-wide columns
// run in the order {4 lg .. 4 lg + 3, 16 + 4 lg .. + 3} in every operand (the order in which an
// MFMA result leaves Q_c in the lanes), which leaves each product's sum unchanged.
template <int W>
struct CtxFrags {
  static constexpr int PV = (W / 16 + 3) / 4;   // W_v tiles per wave
  bf16x8 kt[2][W / 32];   // W_k^T rows 16 t + l16, slice columns 32 kb + 8 lg .. + 7
  bf16x8 bk[W / 32];      // b_k at the same columns
  bf16x8 vw[PV];          // W_v rows g W + 16 tau + l16 (tau = wave + 4 i), columns 8 lg .. + 7
  bf16x4 vb[PV];          // b_v[g W + 16 tau + 4 lg .. + 3]
};

template <int W>
__device__ __forceinline__ void ctx_frags_load(const TinyArgs& a, int l, int g, CtxFrags<W>& f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  const int A = a.A;
  const bf16* kt = a.ck_wt + (size_t)l * TH * A + g * W;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int kb = 0; kb < W / 32; ++kb) f.kt[t][kb] = load8(kt + (size_t)(t * 16 + l16) * A + kb * 32 + lg * 8);
#pragma unroll
  for (int kb = 0; kb < W / 32; ++kb) f.bk[kb] = load8(a.ck_b + (size_t)l * A + g * W + kb * 32 + lg * 8);
#pragma unroll
  for (int i = 0; i < CtxFrags<W>::PV; ++i) {
    int tau = wave + 4 * i;
    tau = tau < W / 16 ? tau : W / 16 - 1;
    const int row = g * W + tau * 16;
    f.vw[i] = load8(a.cv_w + ((size_t)l * A + row + l16) * TH + lg * 8);
    f.vb[i] = *reinterpret_cast<const bf16x4*>(a.cv_b + (size_t)l * A + row + lg * 4);
  }
}

struct CtxBlock {
  bf16x8 h[2];   // row 32 blk + 16 sub + l16, columns {4 lg .. + 3, 16 + 4 lg .. + 3}
  f32x4 r[2];    // factors (r * scale * log2 e) of keys 32 blk + 16 sub + 4 lg .. + 3
};

// rows past Lc read row 0, blocks past the last read block 0 (scores masked, values weighed by 0)
__device__ __forceinline__ void ctx_block_load(const TinyArgs& a, int l, int blk, CtxBlock& cb) {
  const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
  const int bb = blk * 32 < a.Lcp ? blk : 0;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    int kk = bb * 32 + sub * 16 + l16;
    kk = kk < a.Lc ? kk : 0;
    const bf16* row = a.ctx_emb + (size_t)kk * a.ctx_emb_ld;
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row + 4 * lg);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(row + 16 + 4 * lg);
    cb.h[sub] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    cb.r[sub] = *reinterpret_cast<const f32x4*>(a.ctx_rs + (size_t)l * a.Lcp + bb * 32 + sub * 16 + 4 * lg);
  }
}

// Folded queries, online softmax over the context blocks (round-robin over the waves, the wave's
// rows staged in its tile for the transposed reads of Z^T += H^T P^T), the waves merged in order
// into Z (hi + lo bf16 in LDS), then O^T = W_v Z^T + b_v of the slice's dims -> sm.o.
template <int W, int NCB>
__device__ __forceinline__ void attend_ctx(const TinyArgs& a, TinySmem<W, NCB>& sm, int l, const CtxFrags<W>& f,
                                           CtxBlock& cur) {
  constexpr int WK = W / 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  const int S = a.S, n = a.Lc, nblk = (n + 31) / 32;
  const int dsh = __builtin_ctz(a.DH), nc = (W >> dsh) * S;
  // Q_c^T (hi, lo) and beta_c of column c = cb * 16 + l16 = (head hh, token s)
  bf16x8 qh[NCB], ql[NCB];
  float beta[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int c = cb * 16 + l16, hh = c / S, s = c - hh * S;
    f32x4 d0 = f32x4{0.f, 0.f, 0.f, 0.f}, d1 = d0;
    float bs = 0.f;
#pragma unroll
    for (int kb = 0; kb < WK; ++kb) {
      const int c0 = kb * 32 + lg * 8;
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(&sm.q[c < nc ? s : 0][c0]);
      const bf16x8 qf = (c < nc && (c0 >> dsh) == hh) ? x : zero8();
#pragma unroll
      for (int e = 0; e < 8; ++e) bs += to_f(qf[e]) * to_f(f.bk[kb][e]);
      d0 = mfma16(f.kt[0][kb], qf, d0);   // Q_c[4 lg + e]
      d1 = mfma16(f.kt[1][kb], qf, d1);   // Q_c[16 + 4 lg + e]
    }
    beta[cb] = group4_sum(bs);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qh[cb][e] = to_bf(d0[e]);
      ql[cb][e] = to_bf(d0[e] - to_f(qh[cb][e]));
      qh[cb][4 + e] = to_bf(d1[e]);
      ql[cb][4 + e] = to_bf(d1[e] - to_f(qh[cb][4 + e]));
    }
  }
  float m[NCB], lsum[NCB];
  f32x4 acc[2][NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    m[cb] = -INFINITY;
    lsum[cb] = 0.f;
    acc[0][cb] = acc[1][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  bf16(*ht)[48] = reinterpret_cast<bf16(*)[48]>(&sm.vt[wave][0][0]);   // 32 rows x 32 (+ 16 pad)
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  for (int blk = wave; blk < nblk; blk += 4) {
    CtxBlock nx;
    if (blk + 4 < nblk) ctx_block_load(a, l, blk + 4, nx);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      *reinterpret_cast<bf16x4*>(&ht[sub * 16 + l16][4 * lg]) = __builtin_shufflevector(cur.h[sub], cur.h[sub], 0, 1, 2, 3);
      *reinterpret_cast<bf16x4*>(&ht[sub * 16 + l16][16 + 4 * lg]) =
          __builtin_shufflevector(cur.h[sub], cur.h[sub], 4, 5, 6, 7);
    }
    bf16x8 pf[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      float sc[2][4];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        f32x4 d = mfma16(cur.h[sub], qh[cb], f32x4{0.f, 0.f, 0.f, 0.f});
        d = mfma16(cur.h[sub], ql[cb], d);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kk = blk * 32 + sub * 16 + lg * 4 + e;
          sc[sub][e] = kk < n ? (d[e] + beta[cb]) * cur.r[sub][e] : -INFINITY;
        }
      }
      float alpha;
      if (softmax_block(sc, m[cb], lsum[cb], pf[cb], alpha)) {
        acc[0][cb] *= alpha;
        acc[1][cb] *= alpha;
      }
    }
    // H^T fragments: rows = columns 16 t + l16, k = keys {4 lg .. + 3, 16 + 4 lg .. + 3}
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = lg * 4 + (l16 >> 2), col = t * 16 + 4 * (l16 & 3);
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&ht[key][col]);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&ht[key + 16][col]);
      const s16x8 h8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      const bf16x8 hf = __builtin_bit_cast(bf16x8, h8);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) acc[t][cb] = mfma16(hf, pf[cb], acc[t][cb]);
    }
    if (blk + 4 < nblk) cur = nx;
  }
  // merge the waves' states through LDS, in wave order
  if (lg == 0) {
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      sm.u.mg.m[wave][cb * 16 + l16] = m[cb];
      sm.u.mg.l[wave][cb * 16 + l16] = lsum[cb];
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
      *reinterpret_cast<f32x4*>(&sm.u.mg.acc[wave][cb * 16 + l16][t * 16 + lg * 4]) = acc[t][cb];
  lds_barrier();
  // Z of every column (8 of its 32 entries per thread) as hi + lo bf16; the wave tiles are free
  bf16(*zh)[40] = reinterpret_cast<bf16(*)[40]>(&sm.vt[0][0][0]);
  bf16(*zl)[40] = zh + NCB * 16;
  if (threadIdx.x < NCB * 64) {
    const int c = threadIdx.x >> 2, j0 = (threadIdx.x & 3) * 8;
    float mw[4], mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = sm.u.mg.m[w][c];
      mx = fmaxf(mx, mw[w]);
    }
    const float ms = mx == -INFINITY ? 0.f : mx;
    float fw[4], den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      fw[w] = __builtin_amdgcn_exp2f(mw[w] - ms);
      den += fw[w] * sm.u.mg.l[w][c];
    }
    f32x4 z0 = f32x4{0.f, 0.f, 0.f, 0.f}, z1 = z0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      z0 += fw[w] * *reinterpret_cast<const f32x4*>(&sm.u.mg.acc[w][c][j0]);
      z1 += fw[w] * *reinterpret_cast<const f32x4*>(&sm.u.mg.acc[w][c][j0 + 4]);
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    bf16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float u = z0[e] * inv, v = z1[e] * inv;
      hi[e] = to_bf(u);
      lo[e] = to_bf(u - to_f(hi[e]));
      hi[4 + e] = to_bf(v);
      lo[4 + e] = to_bf(v - to_f(hi[4 + e]));
    }
    *reinterpret_cast<bf16x8*>(&zh[c][j0]) = hi;
    *reinterpret_cast<bf16x8*>(&zl[c][j0]) = lo;
  }
  lds_barrier();
  // O^T = W_v Z^T + b_v: dims 16 tau + 4 lg + e of column cb * 16 + l16, kept where the dims
  // belong to the column's head (4 consecutive dims never straddle a head: head_dim % 8 == 0)
#pragma unroll
  for (int i = 0; i < CtxFrags<W>::PV; ++i) {
    const int tau = wave + 4 * i;
    if (tau < W / 16) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const int c = cb * 16 + l16, hh = c / S, s = c - hh * S, d0 = tau * 16 + lg * 4;
        f32x4 d = mfma16(f.vw[i], *reinterpret_cast<const bf16x8*>(&zh[c][lg * 8]), f32x4{0.f, 0.f, 0.f, 0.f});
        d = mfma16(f.vw[i], *reinterpret_cast<const bf16x8*>(&zl[c][lg * 8]), d);
        if (c < nc && (d0 >> dsh) == hh) {
          bf16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = to_bf(d[e] + to_f(f.vb[i][e]));
          *reinterpret_cast<bf16x4*>(&sm.o[s][d0]) = o;
        }
      }
    }
  }
  lds_barrier();
}

// The slice's share of an o projection: part[s][n] = sum_d o[s][d] Wo[n][g W + d] (waves 0, 1:
// one 16-row tile of the 32 outputs each, all W / 32 k-blocks).
template <int W, int NCB>
__device__ __forceinline__ void oproj_store(TinySmem<W, NCB>& sm, const bf16x8 (&of)[W / 32], float* part, int S) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  if (wave >= 2) return;
  f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < W / 32; ++kb)
    d = mfma16(of[kb], *reinterpret_cast<const bf16x8*>(&sm.o[l16][kb * 32 + lg * 8]), d);
  if (l16 < S) *reinterpret_cast<f32x4*>(part + l16 * TH + wave * 16 + lg * 4) = d;
}

template <int W>
__device__ __forceinline__ void oproj_load(const bf16* w, int A, int g, bf16x8 (&of)[W / 32]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lg = lane >> 4;
  const int t = wave & 1;
#pragma unroll
  for (int kb = 0; kb < W / 32; ++kb) of[kb] = load8(w + (size_t)(t * 16 + l16) * A + g * W + kb * 32 + lg * 8);
}

// Normalise (RMS over A columns from ss[which]) a slice of raw rows into dst (bf16), with the
// reference's rounding (bf16 before the weight), optionally rotating pairs by the 1-D table, or
// weighting the rounded result by a second vector nw2 (the key norm weight a folded query carries).
template <int W, int NCB>
__device__ __forceinline__ void norm_slice(const TinyArgs& a, TinySmem<W, NCB>& sm, int which, int rawcol,
                                           bf16 (*dst)[W + 8], const bf16* nw, bool rope, const bf16* nw2 = nullptr) {
  constexpr int CPR = W / 8;
  const int S = a.S;
  for (int idx = threadIdx.x; idx < S * CPR; idx += 256) {
    const int s = idx / CPR, d0 = (idx - s * CPR) * 8;
    const float r = rsqrtf(sm.ss[which][s] / (float)a.A + a.eps);
    const bf16x8 w8 = load8(nw + d0);
    const bf16x8 w2 = nw2 != nullptr ? load8(nw2 + d0) : zero8();
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = to_f(to_bf(sm.u.raw[s][rawcol + d0 + e] * r)) * to_f(w8[e]);
    if (nw2 != nullptr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = to_f(to_bf(y[e])) * to_f(w2[e]);
    }
    if (rope) {
      const int j0 = (d0 % a.DH) / 2, hd2 = a.DH / 2;
      const f32x4 cs = *reinterpret_cast<const f32x4*>(a.rcos + s * hd2 + j0);
      const f32x4 sn = *reinterpret_cast<const f32x4*>(a.rsin + s * hd2 + j0);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float u = to_f(to_bf(y[2 * p])), v = to_f(to_bf(y[2 * p + 1]));
        y[2 * p] = u * cs[p] - v * sn[p];
        y[2 * p + 1] = u * sn[p] + v * cs[p];
      }
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf(y[e]);
    *reinterpret_cast<bf16x8*>(&dst[s][d0]) = o;
  }
}

// direct sums of squares over the slice (one slice covers all A columns)
template <int W, int NCB>
__device__ __forceinline__ void direct_sumsq(TinySmem<W, NCB>& sm, int which, int rawcol, int S) {
  const int s = threadIdx.x >> 4, j = threadIdx.x & 15;
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < W / 16; ++e) {
    const float x = sm.u.raw[s][rawcol + j * (W / 16) + e];
    acc += x * x;
  }
  acc = row16_sum(acc);
  if (j == 0 && s < S) sm.ss[which][s] = acc;
}

// ---------------------------------------------------------------------------------------
// Fixed-order sum over the G slices of the fp32 partials part[b, g, s, 0..32): thread
// (gi, slot) adds slices gi, gi + NGI, gi + 2 NGI, ... of 4 consecutive columns of one row, and
// the NGI <= 4 sums meet in sm.u.f.red[gi] (the row op then adds them in gi order).  Every
// workgroup of a batch row performs the same sums in the same order.
struct PartLoads {
  f32x4 v[8];
};

// loads of round `round` that any thread needs (the same count for the whole workgroup)
__device__ __forceinline__ int part_loads(int G, int NGI, int round) {
  return min(8, (G + NGI - 1) / NGI - 8 * round);
}

__device__ __forceinline__ void part_issue(const float* part, int b, int G, int S, int round, PartLoads& pl) {
  const int NV = S * 8, NGI = min(4, 256 / NV), tid = threadIdx.x, nu = part_loads(G, NGI, round);
  const int gi = tid / NV, slot = tid - gi * NV, s = slot >> 3, n4 = slot & 7;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (u < nu) {
      const int g = gi + NGI * (8 * round + u);
      const bool ok = gi < NGI && g < G;
      // out-of-range slots read slice 0's (finite) row; part_reduce weighs them by 0
      pl.v[u] = *reinterpret_cast<const f32x4*>(part + (((size_t)b * G + (ok ? g : 0)) * S + (ok ? s : 0)) * TH +
                                                4 * (ok ? n4 : 0));
    }
  }
}

template <int W, int NCB>
__device__ __forceinline__ void part_reduce(TinySmem<W, NCB>& sm, const float* part, int b, int G, int S,
                                            PartLoads& pl) {
  const int NV = S * 8, NGI = min(4, 256 / NV), tid = threadIdx.x;
  const int gi = tid / NV, slot = tid - gi * NV, s = slot >> 3, n4 = slot & 7;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int round = 0; round * 8 * NGI < G; ++round) {
    if (round > 0) part_issue(part, b, G, S, round, pl);
    const int nu = part_loads(G, NGI, round);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int g = gi + NGI * (8 * round + u);
      if (u < nu) acc += pl.v[u] * ((gi < NGI && g < G) ? 1.0f : 0.0f);
    }
  }
  if (gi < NGI) *reinterpret_cast<f32x4*>(&sm.u.f.red[gi][s][4 * n4]) = acc;
}

// sum of the reduced partials of element (s_r, 2 j_r + c)
template <int W, int NCB>
__device__ __forceinline__ float part_sum(TinySmem<W, NCB>& sm, int S, int s, int n) {
  const int NGI = min(4, 256 / (S * 8));
  float y = sm.u.f.red[0][s][n];
  for (int gi = 1; gi < NGI; ++gi) y += sm.u.f.red[gi][s][n];
  return y;
}

// ---------------------------------------------------------------------------------------
// Small matrices staged in LDS: the encoder and head weights (scalar loads at phase start).
struct SmallW {
  bf16 e[4], h[4];
};

__device__ __forceinline__ void small_load(const TinyArgs& a, SmallW& w) {
  const int n = TH * a.Da;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = threadIdx.x + 256 * i;
    w.e[i] = a.enc_w[idx < n ? idx : 0];
    w.h[i] = a.head_w[idx < n ? idx : 0];
  }
}

template <int W, int NCB>
__device__ __forceinline__ void small_store(const TinyArgs& a, TinySmem<W, NCB>& sm, const SmallW& w) {
  const int n = TH * a.Da;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = threadIdx.x + 256 * i;
    if (idx < n) {
      sm.ew[idx] = w.e[i];
      sm.hw[idx] = w.h[i];
    }
  }
}

// the chunk update of step tt (head + Euler) from the rows in sm.x: lat = lat_old + delta v.
// lat_old is this thread's element (s, j) = (tid / Da, tid % Da), loaded early.
template <int W, int NCB>
__device__ __forceinline__ void head_euler(const TinyArgs& a, TinySmem<W, NCB>& sm, float lat_old, float hb_j,
                                           float delta, float* dst) {
  const int idx = threadIdx.x, Da = a.Da;
  if (idx < a.S * Da) {
    const int s = idx / Da, j = idx - s * Da;
    float v = 0.f;
#pragma unroll 8
    for (int n = 0; n < TH; ++n) v += sm.x[s][n] * to_f(sm.hw[j * TH + n]);
    const float y = lat_old + delta * (v + hb_j);
    sm.lat[s][j] = y;
    if (dst != nullptr) dst[idx] = y;
  }
}

// x = lat W_enc^T + b_enc (fp32) into sm.x
template <int W, int NCB>
__device__ __forceinline__ void encoder(const TinyArgs& a, TinySmem<W, NCB>& sm, bf16x2 eb) {
  const int s = threadIdx.x >> 4, j = threadIdx.x & 15, Da = a.Da;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 2 * j + c;
    float y = to_f(eb[c]);
    for (int q = 0; q < Da; ++q) y += sm.lat[s][q] * to_f(sm.ew[n * Da + q]);
    sm.x[s][n] = s < a.S ? y : 0.f;
  }
}

// ---------------------------------------------------------------------------------------
// Phase: self (MoT joint) attention sub-block of block l at step t.
template <int W, int NCB>
__device__ __forceinline__ void phase_self(const TinyArgs& a, TinySmem<W, NCB>& sm, int g, int b, int t, int l) {
  constexpr int WT = W / 16;
  using SF = SliceFrags<W>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int S = a.S, A = a.A, L = a.L, G = a.G;
  const int s_r = tid >> 4, j_r = tid & 15;   // row-op mapping
  const bool first = (t == 0 && l == 0);
  const bool step0 = (l == 0);                // the first block of a step: head, Euler, encoder
  const int lp = l == 0 ? L - 1 : l - 1, tp = l == 0 ? t - 1 : t;
  const size_t rows = (size_t)a.B * S;

  // ---- loads that do not depend on the rows
  SF qkv;
  {
    const bf16* w = a.qkv_w + (size_t)l * 3 * A * TH;
    const bf16* bb = a.qkv_b + (size_t)l * 3 * A;
#pragma unroll
    for (int i = 0; i < SF::PW; ++i) {
      int tau = wave + 4 * i;
      tau = tau < SF::NT ? tau : SF::NT - 1;
      const int which = tau / WT, r = tau - which * WT, row = which * A + g * W + r * 16;
      qkv.w[i] = load8(w + (size_t)(row + l16) * TH + lg * 8);
      qkv.b[i] = *reinterpret_cast<const bf16x4*>(bb + row + lg * 4);
    }
  }
  FfnFrags ff;
  if (!first) ffn_load(a, lp, ff);
  SmallW sw;
  if (step0) small_load(a, sw);
  KvSrc src;
  src.n0 = a.Sv;
  src.n1 = S;
  src.rs0 = a.v_rs;
  src.k0 = a.Sv > 0 ? a.vk[l] + b * a.v_bs + g * W : nullptr;
  src.v0 = a.Sv > 0 ? a.vv[l] + b * a.v_bs + g * W : nullptr;
  const bool pre = a.Sv > wave * 32;   // the wave's first block holds video keys (action rows patched in later)
  // row-op operands
  const bf16* modt = a.mods + ((size_t)t * L + l) * 6 * TH;
  const RowMod m1 = row_mod_load(modt, modt + TH);   // shift_msa, scale_msa
  RowMod m2;
  bf16x2 cob, b2, gmlp, eb;
  float yv[2] = {0.f, 0.f};
  PartLoads pl;
  // the previous cross phase split the context (one 32-wide slice): its splits, merged here
  const bool xsplit = W == 32 && a.KS > 1;
  XSplit xs;
  bf16x8 ofc[W / 32];
  float lat_old = 0.f, hbj = 0.f, delta = 0.f;
  if (!first) {
    const bf16* modp = a.mods + ((size_t)tp * L + lp) * 6 * TH;
    m2 = row_mod_load(modp + 3 * TH, modp + 4 * TH);   // shift_mlp, scale_mlp
    gmlp = *reinterpret_cast<const bf16x2*>(modp + 5 * TH + 2 * j_r);
    cob = *reinterpret_cast<const bf16x2*>(a.co_b + (size_t)lp * TH + 2 * j_r);
    b2 = *reinterpret_cast<const bf16x2*>(a.ff2_b + (size_t)lp * TH + 2 * j_r);
    const int sr = s_r < S ? s_r : 0;
    const f32x2 y = *reinterpret_cast<const f32x2*>(a.xb + ((size_t)b * S + sr) * TH + 2 * j_r);
    yv[0] = y[0];
    yv[1] = y[1];
    if (xsplit) {
      xsplit_issue<W>(a, b, xs);
      oproj_load<W>(a.co_w + (size_t)lp * TH * A, A, 0, ofc);
    } else {
      part_issue(a.part_c, b, G, S, 0, pl);
    }
  }
  if (step0) {
    eb = *reinterpret_cast<const bf16x2*>(a.enc_b + 2 * j_r);
    const int Da = a.Da, e = tid < S * Da ? tid : 0;
    if (first) {
      lat_old = to_f(a.noise[(size_t)b * S * Da + e]);
    } else {
      lat_old = a.lat[(size_t)((t - 1) & 1) * rows * Da + (size_t)b * S * Da + e];
      hbj = to_f(a.head_b[e % Da]);
      delta = to_f(a.deltas[t - 1]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the rows entering block l
  if (step0) small_store(a, sm, sw);
  if (!first) {
    if (xsplit)
      xsplit_merge(a, sm, xs, ofc);
    else
      part_reduce(sm, a.part_c, b, G, S, pl);
    lds_barrier();
    const float x0 = yv[0] + (to_f(cob[0]) + part_sum(sm, S, s_r, 2 * j_r));
    const float x1 = yv[1] + (to_f(cob[1]) + part_sum(sm, S, s_r, 2 * j_r + 1));
    lds_barrier();
    sm.x[s_r][2 * j_r] = s_r < S ? x0 : 0.f;
    sm.x[s_r][2 * j_r + 1] = s_r < S ? x1 : 0.f;
    lds_barrier();
    row_norm(sm, S, a.eps, m2, true);
    lds_barrier();
    ffn_apply(a, sm, ff, b2, gmlp);
  }
  // second stage of the early loads (after the FFN fragments are consumed)
  GramFrags gf;
  if (G > 1) gram_load(a, l, wave & 1, gf);
  bf16x8 of[W / 32];
  oproj_load<W>(a.o_w + (size_t)l * TH * A, A, g, of);
  KvBlock<W> kv;
  if (pre) kv_load_global<W>(src, wave, kv);
  __builtin_amdgcn_sched_barrier(0);
  if (step0) {
    float* dst = g == 0 ? a.lat + (size_t)(t & 1) * rows * a.Da + (size_t)b * S * a.Da : nullptr;
    if (first) {
      if (tid < S * a.Da) {
        sm.lat[tid / a.Da][tid % a.Da] = lat_old;
        if (dst != nullptr) dst[tid] = lat_old;
      }
    } else {
      head_euler(a, sm, lat_old, hbj, delta, dst);
    }
    lds_barrier();
    encoder(a, sm, eb);
    lds_barrier();
  }
  if (g == 0 && s_r < S)
    *reinterpret_cast<f32x2*>(a.xa + ((size_t)b * S + s_r) * TH + 2 * j_r) = f32x2{sm.x[s_r][2 * j_r], sm.x[s_r][2 * j_r + 1]};
  row_norm(sm, S, a.eps, m1, true);
  lds_barrier();

  // ---- q, k, v of the slice (+ the rows' sums of squares over all A columns)
  {
    const bf16x8 hf = hb_frag(sm);
#pragma unroll
    for (int i = 0; i < SF::PW; ++i) {
      const int tau = wave + 4 * i;
      if (tau < SF::NT) {
        const int which = tau / WT, r = tau - which * WT;
        const f32x4 d = mfma16(qkv.w[i], hf, f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = d[e] + to_f(qkv.b[i][e]);
        *reinterpret_cast<f32x4*>(&sm.u.raw[l16][which * W + r * 16 + lg * 4]) = y;
      }
    }
    if (G > 1 && wave < 2) gram_sumsq(sm, gf, wave, S);
  }
  lds_barrier();
  if (G == 1) {
    direct_sumsq(sm, 0, 0, S);
    direct_sumsq(sm, 1, W, S);
    lds_barrier();
  }
  norm_slice(a, sm, 0, 0, sm.q, a.nq_w + (size_t)l * A + g * W, true);
  norm_slice(a, sm, 1, W, sm.k, a.nk_w + (size_t)l * A + g * W, true);
  for (int idx = tid; idx < S * (W / 8); idx += 256) {
    const int s = idx / (W / 8), d0 = (idx - s * (W / 8)) * 8;
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf(sm.u.raw[s][2 * W + d0 + e]);
    *reinterpret_cast<bf16x8*>(&sm.v[s][d0]) = o;
  }
  lds_barrier();

  // ---- attention over [video K/V ; action K/V], then the slice's o-projection partial
  attend<1>(a, sm, src, a.mask, a.mask_rs, kv, pre);
  oproj_store(sm, of, a.part_s + ((size_t)b * G + g) * S * TH, S);
}

// Phase: cross-attention sub-block of block l at step t.
template <int W, int NCB>
__device__ __forceinline__ void phase_cross(const TinyArgs& a, TinySmem<W, NCB>& sm, int g, int ks, int b, int t,
                                            int l) {
  constexpr int WT = W / 16, PW = (WT + 3) / 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int S = a.S, A = a.A, L = a.L, G = a.G;
  const int s_r = tid >> 4, j_r = tid & 15;

  bf16x8 qw[PW];
  bf16x4 qb[PW];
  {
    const bf16* w = a.cq_w + (size_t)l * A * TH;
    const bf16* bb = a.cq_b + (size_t)l * A;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      int tau = wave + 4 * i;
      tau = tau < WT ? tau : WT - 1;
      const int row = g * W + tau * 16;
      qw[i] = load8(w + (size_t)(row + l16) * TH + lg * 8);
      qb[i] = *reinterpret_cast<const bf16x4*>(bb + row + lg * 4);
    }
  }
  GramFrags gf;
  if (G > 1) gram_load(a, l, 2, gf);
  bf16x8 of[W / 32];
  oproj_load<W>(a.co_w + (size_t)l * TH * A, A, g, of);
  // every wave's first context block is loaded, also by a wave without one (rows past Lc read
  // row 0): an unconditional load keeps the block in registers where the attention picks it up
  constexpr bool folded = W > TH;   // attention in the space of the 32-wide context rows
  KvBlock<W> kv;
  KvSrc src;
  CtxFrags<W> cf;
  CtxBlock cblk;
  if constexpr (folded) {
    ctx_frags_load<W>(a, l, g, cf);
    ctx_block_load(a, l, wave, cblk);
  } else {
    // split ks of KS: whole 32-key blocks [ks per, (ks + 1) per) (every split holds keys)
    const int nblk = (a.Lc + 31) / 32, per = (nblk + a.KS - 1) / a.KS, key0 = ks * per * 32;
    src.n0 = min(a.Lc, key0 + per * 32) - key0;
    src.n1 = 0;
    src.rs0 = a.ctx_ld;
    src.k0 = a.ctxkv + (size_t)key0 * a.ctx_ld + (size_t)l * 2 * A + g * W;
    src.v0 = a.ctxkv + (size_t)key0 * a.ctx_ld + (size_t)l * 2 * A + A + g * W;
    kv_load_global<W>(src, wave, kv);
  }
  const bf16* modt = a.mods + ((size_t)t * L + l) * 6 * TH;
  const bf16x2 gmsa = *reinterpret_cast<const bf16x2*>(modt + 2 * TH + 2 * j_r);
  const bf16x2 ob = *reinterpret_cast<const bf16x2*>(a.o_b + (size_t)l * TH + 2 * j_r);
  const RowMod n3 = row_mod_load(a.n3_w + (size_t)l * TH, a.n3_b + (size_t)l * TH);
  const int sr = s_r < S ? s_r : 0;
  const f32x2 xv = *reinterpret_cast<const f32x2*>(a.xa + ((size_t)b * S + sr) * TH + 2 * j_r);
  PartLoads pl;
  part_issue(a.part_s, b, G, S, 0, pl);
  __builtin_amdgcn_sched_barrier(0);

  part_reduce(sm, a.part_s, b, G, S, pl);
  lds_barrier();
  {
    const float o0 = to_f(ob[0]) + part_sum(sm, S, s_r, 2 * j_r);
    const float o1 = to_f(ob[1]) + part_sum(sm, S, s_r, 2 * j_r + 1);
    const float x0 = xv[0] + to_f(gmsa[0]) * o0, x1 = xv[1] + to_f(gmsa[1]) * o1;
    sm.x[s_r][2 * j_r] = s_r < S ? x0 : 0.f;
    sm.x[s_r][2 * j_r + 1] = s_r < S ? x1 : 0.f;
    if (g == 0 && ks == 0 && s_r < S)
      *reinterpret_cast<f32x2*>(a.xb + ((size_t)b * S + s_r) * TH + 2 * j_r) = f32x2{x0, x1};
  }
  lds_barrier();
  row_norm(sm, S, a.eps, n3, false);
  lds_barrier();
  {
    const bf16x8 hf = hb_frag(sm);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int tau = wave + 4 * i;
      if (tau < WT) {
        const f32x4 d = mfma16(qw[i], hf, f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = d[e] + to_f(qb[i][e]);
        *reinterpret_cast<f32x4*>(&sm.u.raw[l16][tau * 16 + lg * 4]) = y;
      }
    }
    if (G > 1 && wave == 0) gram_sumsq(sm, gf, 2, S);
  }
  lds_barrier();
  if (G == 1) {
    direct_sumsq(sm, 2, 0, S);
    lds_barrier();
  }
  norm_slice(a, sm, 2, 0, sm.q, a.cnq_w + (size_t)l * A + g * W, false,
             folded ? a.cnk_w + (size_t)l * A + g * W : nullptr);
  lds_barrier();
  if constexpr (folded) {
    attend_ctx<W, NCB>(a, sm, l, cf, cblk);
  } else if (a.KS > 1) {
    // the split's state; the next phase merges the splits and projects
    attend<3>(a, sm, src, nullptr, 0, kv, true, a.part_x + (size_t)(b * a.KS + ks) * 32 * (W + 4));
    return;
  } else {
    attend<3>(a, sm, src, nullptr, 0, kv, true);
  }
  oproj_store(sm, of, a.part_c + ((size_t)b * G + g) * S * TH, S);
}

// Phase: the last block's FFN, the head and the last Euler update -> out.
template <int W, int NCB>
__device__ __forceinline__ void phase_final(const TinyArgs& a, TinySmem<W, NCB>& sm, int b) {
  const int tid = threadIdx.x, j_r = tid & 15, s_r = tid >> 4;
  const int S = a.S, L = a.L, G = a.G, T = a.T, lp = L - 1, tp = T - 1;
  const size_t rows = (size_t)a.B * S;
  FfnFrags ff;
  ffn_load(a, lp, ff);
  SmallW sw;
  small_load(a, sw);
  const bf16* modp = a.mods + ((size_t)tp * L + lp) * 6 * TH;
  const RowMod m2 = row_mod_load(modp + 3 * TH, modp + 4 * TH);
  const bf16x2 gmlp = *reinterpret_cast<const bf16x2*>(modp + 5 * TH + 2 * j_r);
  const bf16x2 cob = *reinterpret_cast<const bf16x2*>(a.co_b + (size_t)lp * TH + 2 * j_r);
  const bf16x2 b2 = *reinterpret_cast<const bf16x2*>(a.ff2_b + (size_t)lp * TH + 2 * j_r);
  const int sr = s_r < S ? s_r : 0;
  const f32x2 y = *reinterpret_cast<const f32x2*>(a.xb + ((size_t)b * S + sr) * TH + 2 * j_r);
  PartLoads pl;
  const bool xsplit = W == 32 && a.KS > 1;
  XSplit xs;
  bf16x8 ofc[W / 32];
  if (xsplit) {
    xsplit_issue<W>(a, b, xs);
    oproj_load<W>(a.co_w + (size_t)lp * TH * a.A, a.A, 0, ofc);
  } else {
    part_issue(a.part_c, b, G, S, 0, pl);
  }
  const int Da = a.Da, e = tid < S * Da ? tid : 0;
  const float lat_old = a.lat[(size_t)(tp & 1) * rows * Da + (size_t)b * S * Da + e];
  const float hbj = to_f(a.head_b[e % Da]);
  const float delta = to_f(a.deltas[tp]);
  __builtin_amdgcn_sched_barrier(0);
  small_store(a, sm, sw);
  if (xsplit)
    xsplit_merge(a, sm, xs, ofc);
  else
    part_reduce(sm, a.part_c, b, G, S, pl);
  lds_barrier();
  const float x0 = y[0] + (to_f(cob[0]) + part_sum(sm, S, s_r, 2 * j_r));
  const float x1 = y[1] + (to_f(cob[1]) + part_sum(sm, S, s_r, 2 * j_r + 1));
  lds_barrier();
  sm.x[s_r][2 * j_r] = s_r < S ? x0 : 0.f;
  sm.x[s_r][2 * j_r + 1] = s_r < S ? x1 : 0.f;
  lds_barrier();
  row_norm(sm, S, a.eps, m2, true);
  lds_barrier();
  ffn_apply(a, sm, ff, b2, gmlp);
  head_euler(a, sm, lat_old, hbj, delta, a.out + (size_t)b * S * Da);
}

// One phase per launch, one kernel per phase kind.  A loop over phases inside one kernel lets the
// compiler hoist every lane's addresses of every phase out of the loop and keep them live
// (spilling to scratch); one kernel for all three kinds loads every kind's pointers from the
// kernel arguments at entry and spills scalar registers.
template <int W, int NCB>
__global__ __launch_bounds__(256, 1) void tiny_self_kernel(TinyArgs a) {
  __shared__ TinySmem<W, NCB> sm;
  const int per = 2 * a.L, t = a.p0 / per, l = (a.p0 - t * per) >> 1;
  phase_self(a, sm, blockIdx.x, blockIdx.y, t, l);
}

template <int W, int NCB>
__global__ __launch_bounds__(256, 1) void tiny_cross_kernel(TinyArgs a) {
  __shared__ TinySmem<W, NCB> sm;
  const int per = 2 * a.L, t = a.p0 / per, l = (a.p0 - t * per) >> 1;
  // (with context splits the slice is the only one: blockIdx.x numbers the splits)
  phase_cross(a, sm, a.KS > 1 ? 0 : (int)blockIdx.x, a.KS > 1 ? (int)blockIdx.x : 0, blockIdx.y, t, l);
}

template <int W, int NCB>
__global__ __launch_bounds__(256, 1) void tiny_final_kernel(TinyArgs a) {
  __shared__ TinySmem<W, NCB> sm;
  phase_final(a, sm, blockIdx.y);
}

// The context keys' factors r * scale * log2 e, r = rsqrt(mean_j k_j^2 + eps) over all A columns
// of k = W_k h + b_k, from the cross key weight's Gram form h G h + 2 h.c + |b|^2 (G = hi + lo):
// one thread per (key, layer); keys past Lc (to the 32-key block) read row 0.
__global__ __launch_bounds__(256) void tiny_ctx_rs_kernel(TinyArgs a) {
  __shared__ float gs[TH][TH + 1];
  __shared__ float cs[TH];
  const int l = blockIdx.y, tid = threadIdx.x;
  const bf16* gh = a.gram + (size_t)(l * 4 + 3) * 2 * TH * TH;
  for (int i = tid; i < TH * TH; i += 256) gs[i / TH][i % TH] = to_f(gh[i]) + to_f(gh[TH * TH + i]);
  if (tid < TH) cs[tid] = 2.0f * a.gram_c[(size_t)(l * 4 + 3) * TH + tid];
  __syncthreads();
  const int key = blockIdx.x * 256 + tid;
  if (key >= a.Lcp) return;
  const bf16* row = a.ctx_emb + (size_t)(key < a.Lc ? key : 0) * a.ctx_emb_ld;
  float h[TH];
#pragma unroll
  for (int i = 0; i < TH / 4; ++i) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(row + 4 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) h[4 * i + e] = to_f(v[e]);
  }
  float q = a.gram_b[l * 4 + 3];
#pragma unroll 4
  for (int i = 0; i < TH; ++i) {
    float gi = cs[i];
#pragma unroll
    for (int j = 0; j < TH; ++j) gi += gs[i][j] * h[j];
    q += h[i] * gi;
  }
  a.ctx_rs[(size_t)l * a.Lcp + key] = rsqrtf(fmaxf(q, 0.f) / (float)a.A + a.eps) * a.scale_log2;
}

template <int W, int NCB>
int launch_tiny(const TinyArgs& a0, int64_t p0, int64_t p1, hipStream_t st) {
  TinyArgs a = a0;
  const int64_t last = 2LL * a.L * a.T;
  void (*self_k)(TinyArgs) = tiny_self_kernel<W, NCB>;
  void (*cross_k)(TinyArgs) = tiny_cross_kernel<W, NCB>;
  void (*final_k)(TinyArgs) = tiny_final_kernel<W, NCB>;
  for (int64_t p = p0; p < p1; ++p) {
    a.p0 = (int)p;
    a.p1 = (int)p + 1;
    if (p == last)
      FAM_LAUNCH(final_k, dim3(1, a.B), dim3(256), 0, st, a);
    else if (p & 1)
      FAM_LAUNCH(cross_k, dim3(a.G * a.KS, a.B), dim3(256), 0, st, a);
    else
      FAM_LAUNCH(self_k, dim3(a.G, a.B), dim3(256), 0, st, a);
    const int rc = fam_host::check_launch("fam_tiny_expert");
    if (rc != FAM_OK) return rc;
  }
  return FAM_OK;
}

}  // namespace
}  // namespace fam

using fam::bf16;

// Checks a descriptor against what the kernels cover and fills the kernel arguments; W (the
// slice) and nc (attention columns per workgroup) for the dispatch.
static int tiny_prepare(const fam_tiny_desc* d, fam::TinyArgs& a, int64_t& W, int64_t& nc, bool need_part_x = true) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_tiny_expert: null descriptor");
  const int64_t B = d->batch, S = d->seq, Hd = d->hidden, NH = d->heads, DH = d->head_dim, F = d->ffn, Da = d->action_dim;
  const int64_t L = d->layers, T = d->steps, Sv = d->video_len, Lc = d->ctx_len;
  const int64_t A = NH * DH;
  W = d->slice > 0 ? d->slice : (A <= 128 ? A : 128);
  FAM_REQUIRE(Hd == 32, FAM_ERR_UNSUPPORTED, "fam_tiny_expert: hidden must be 32 (got %lld)", (long long)Hd);
  FAM_REQUIRE(B >= 1 && B <= 65535 && S >= 1 && S <= 16 && NH >= 1 && L >= 1 && T >= 1 && Lc >= 1 && Sv >= 0,
              FAM_ERR_INVALID_ARG, "fam_tiny_expert: bad shape (B %lld, S %lld, heads %lld, L %lld, T %lld, Lc %lld, Sv %lld)",
              (long long)B, (long long)S, (long long)NH, (long long)L, (long long)T, (long long)Lc, (long long)Sv);
  FAM_REQUIRE(DH >= 8 && DH % 8 == 0 && (W == 32 || W == 64 || W == 128) && W % DH == 0 && A % W == 0,
              FAM_ERR_UNSUPPORTED, "fam_tiny_expert: head_dim %lld / slice %lld / width %lld not supported",
              (long long)DH, (long long)W, (long long)A);
  const int64_t G = A / W;
  nc = (W / DH) * S;
  FAM_REQUIRE(nc <= 32 && G <= 64, FAM_ERR_UNSUPPORTED, "fam_tiny_expert: (slice / head_dim) * S = %lld > 32 or %lld slices > 64",
              (long long)nc, (long long)G);
  FAM_REQUIRE(F >= 32 && F % 32 == 0 && F <= fam::TF, FAM_ERR_UNSUPPORTED,
              "fam_tiny_expert: ffn %lld (need a multiple of 32, <= %d)", (long long)F, fam::TF);
  FAM_REQUIRE(Da >= 1 && Da <= 32 && S * Da <= 256, FAM_ERR_UNSUPPORTED, "fam_tiny_expert: action_dim %lld with %lld tokens",
              (long long)Da, (long long)S);
  FAM_REQUIRE(Sv + S <= (int64_t)1 << 30 && Lc <= (int64_t)1 << 30 && 2 * L * T < (int64_t)1 << 30, FAM_ERR_INVALID_ARG,
              "fam_tiny_expert: sizes too large");
  const bool folded = W > 32;
  const void* need[] = {d->noise, d->mods, d->deltas, d->rope_cos, d->rope_sin, d->enc_w, d->enc_b,
                        d->head_w, d->head_b, d->qkv_w, d->qkv_b, d->nq_w, d->nk_w, d->o_w, d->o_b, d->n3_w, d->n3_b,
                        d->cq_w, d->cq_b, d->cnq_w, d->co_w, d->co_b, d->ff0_w, d->ff0_b, d->ff2_w, d->ff2_b, d->lat,
                        d->xa, d->xb, d->part_s, d->part_c, d->out};
  for (const void* p : need) FAM_REQUIRE(p != nullptr, FAM_ERR_INVALID_ARG, "fam_tiny_expert: a required pointer is null");
  const void* al16[] = {d->mods, d->rope_cos, d->rope_sin, d->qkv_w, d->nq_w, d->nk_w, d->o_w, d->cq_w,
                        d->cnq_w, d->co_w, d->ff0_w, d->ff2_w, d->xa, d->xb, d->part_s, d->part_c};
  for (const void* p : al16) FAM_REQUIRE(fam_host::aligned16(p), FAM_ERR_INVALID_ARG, "fam_tiny_expert: operands must be 16-byte aligned");
  const void* al8[] = {d->qkv_b, d->cq_b, d->ff0_b};
  for (const void* p : al8) FAM_REQUIRE(((uintptr_t)p & 7) == 0, FAM_ERR_INVALID_ARG, "fam_tiny_expert: biases must be 8-byte aligned");
  const void* al4[] = {d->o_b, d->co_b, d->n3_w, d->n3_b, d->ff2_b, d->enc_b};
  for (const void* p : al4) FAM_REQUIRE(((uintptr_t)p & 3) == 0, FAM_ERR_INVALID_ARG, "fam_tiny_expert: row vectors must be 4-byte aligned");
  if (folded) {
    const void* ctx16[] = {d->ck_wt, d->ck_b, d->cnk_w, d->cv_w, d->ctx_rs};
    for (const void* p : ctx16)
      FAM_REQUIRE(p != nullptr && fam_host::aligned16(p), FAM_ERR_INVALID_ARG,
                  "fam_tiny_expert: slice %lld needs ck_wt, ck_b, cnk_w, cv_w and ctx_rs (16-byte aligned)", (long long)W);
    FAM_REQUIRE(d->ctx_emb != nullptr && ((uintptr_t)d->ctx_emb & 7) == 0 && d->ctx_emb_ld >= 32 && d->ctx_emb_ld % 4 == 0 &&
                    d->cv_b != nullptr && ((uintptr_t)d->cv_b & 7) == 0,
                FAM_ERR_INVALID_ARG, "fam_tiny_expert: ctx_emb (8-byte aligned, row stride %lld >= 32, a multiple of 4) and cv_b",
                (long long)d->ctx_emb_ld);
  } else {
    FAM_REQUIRE(d->ctxkv != nullptr && fam_host::aligned16(d->ctxkv), FAM_ERR_INVALID_ARG,
                "fam_tiny_expert: a 32-wide slice reads ctxkv (16-byte aligned)");
    FAM_REQUIRE(d->ctx_ld >= 2 * A * L && d->ctx_ld % 8 == 0, FAM_ERR_INVALID_ARG,
                "fam_tiny_expert: ctx_ld %lld (need >= 2 A L = %lld, a multiple of 8)", (long long)d->ctx_ld, (long long)(2 * A * L));
  }
  FAM_REQUIRE((DH / 2) % 4 == 0, FAM_ERR_UNSUPPORTED, "fam_tiny_expert: head_dim %lld (the rope tables are read 4 pairs at a time)",
              (long long)DH);
  if (G > 1 || folded)
    FAM_REQUIRE(d->gram != nullptr && d->gram_c != nullptr && d->gram_b != nullptr && fam_host::aligned16(d->gram) &&
                    fam_host::aligned16(d->gram_c),
                FAM_ERR_INVALID_ARG, "fam_tiny_expert: %lld slices of %lld need the Gram matrices (16-byte aligned)",
                (long long)G, (long long)W);
  if (Sv > 0) {
    FAM_REQUIRE(d->video_k != nullptr && d->video_v != nullptr && d->video_rs >= A && d->video_rs % 8 == 0 &&
                    d->video_bs % 8 == 0 && (B == 1 || d->video_bs >= Sv * d->video_rs),
                FAM_ERR_INVALID_ARG, "fam_tiny_expert: video K/V tables and strides (row %lld, batch %lld)",
                (long long)d->video_rs, (long long)d->video_bs);
    FAM_REQUIRE(d->video_mask == nullptr || d->mask_rs >= Sv + S, FAM_ERR_INVALID_ARG,
                "fam_tiny_expert: mask row stride %lld < Sv + S", (long long)d->mask_rs);
  }
  a.B = (int)B; a.S = (int)S; a.A = (int)A; a.DH = (int)DH; a.F = (int)F; a.Da = (int)Da; a.L = (int)L; a.T = (int)T;
  a.Sv = (int)Sv; a.Lc = (int)Lc; a.G = (int)G;
  a.eps = d->eps;
  a.scale_log2 = d->scale * 1.4426950408889634f;
  a.noise = (const bf16*)d->noise; a.mods = (const bf16*)d->mods; a.deltas = (const bf16*)d->deltas;
  a.rcos = d->rope_cos; a.rsin = d->rope_sin;
  a.ctxkv = (const bf16*)d->ctxkv; a.ctx_ld = d->ctx_ld;
  a.vk = (const bf16* const*)d->video_k; a.vv = (const bf16* const*)d->video_v;
  a.v_bs = d->video_bs; a.v_rs = d->video_rs;
  a.mask = Sv > 0 ? d->video_mask : nullptr; a.mask_rs = d->mask_rs;
  a.enc_w = (const bf16*)d->enc_w; a.enc_b = (const bf16*)d->enc_b; a.head_w = (const bf16*)d->head_w;
  a.head_b = (const bf16*)d->head_b;
  a.qkv_w = (const bf16*)d->qkv_w; a.qkv_b = (const bf16*)d->qkv_b; a.nq_w = (const bf16*)d->nq_w;
  a.nk_w = (const bf16*)d->nk_w; a.o_w = (const bf16*)d->o_w; a.o_b = (const bf16*)d->o_b;
  a.n3_w = (const bf16*)d->n3_w; a.n3_b = (const bf16*)d->n3_b; a.cq_w = (const bf16*)d->cq_w;
  a.cq_b = (const bf16*)d->cq_b; a.cnq_w = (const bf16*)d->cnq_w; a.co_w = (const bf16*)d->co_w;
  a.co_b = (const bf16*)d->co_b; a.ff0_w = (const bf16*)d->ff0_w; a.ff0_b = (const bf16*)d->ff0_b;
  a.ff2_w = (const bf16*)d->ff2_w; a.ff2_b = (const bf16*)d->ff2_b;
  a.gram = (const bf16*)d->gram; a.gram_c = d->gram_c; a.gram_b = d->gram_b;
  a.lat = d->lat; a.xa = d->xa; a.xb = d->xb; a.part_s = d->part_s; a.part_c = d->part_c; a.out = d->out;
  a.ctx_emb = (const bf16*)d->ctx_emb; a.ctx_emb_ld = d->ctx_emb_ld;
  a.ck_wt = (const bf16*)d->ck_wt; a.ck_b = (const bf16*)d->ck_b; a.cnk_w = (const bf16*)d->cnk_w;
  a.cv_w = (const bf16*)d->cv_w; a.cv_b = (const bf16*)d->cv_b; a.ctx_rs = d->ctx_rs;
  a.Lcp = (int)((Lc + 31) / 32 * 32);
  // context splits of the cross phase: one 32-wide slice and rows few enough that more
  // workgroups find idle CUs (<= 8 splits of >= 4 blocks of 32 keys; every split holds keys)
  int64_t KS = 1;
  if (G == 1 && W == 32) {
    const int64_t nblk = (Lc + 31) / 32;
    int64_t want = d->key_splits > 0 ? d->key_splits
                                     : std::min<int64_t>(fam::TKS, std::max<int64_t>(1, fam_host::device_cus() / B));
    want = std::max<int64_t>(1, std::min<int64_t>({want, (int64_t)fam::TKS, d->key_splits > 0 ? nblk : nblk / 4}));
    const int64_t per = (nblk + want - 1) / want;
    KS = (nblk + per - 1) / per;
  } else {
    FAM_REQUIRE(d->key_splits <= 1, FAM_ERR_UNSUPPORTED,
                "fam_tiny_expert: context splits need one 32-wide slice (slice %lld, %lld slices)", (long long)W,
                (long long)G);
  }
  if (KS > 1 && need_part_x)
    FAM_REQUIRE(d->part_x != nullptr && fam_host::aligned16(d->part_x), FAM_ERR_INVALID_ARG,
                "fam_tiny_expert: %lld context splits need part_x (B * %lld * 32 * (slice + 4) floats, 16-byte aligned)",
                (long long)KS, (long long)KS);
  a.KS = (int)KS;
  a.part_x = d->part_x;
  a.p0 = a.p1 = 0;
  return FAM_OK;
}

extern "C" int fam_tiny_key_splits(const fam_tiny_desc* d) {
  fam::TinyArgs a;
  int64_t W = 0, nc = 0;
  const int rc = tiny_prepare(d, a, W, nc, false);
  return rc != FAM_OK ? -rc : a.KS;
}

extern "C" int fam_tiny_expert(const fam_tiny_desc* d, int64_t phase_begin, int64_t phase_end, void* stream) {
  fam::TinyArgs a;
  int64_t W = 0, nc = 0;
  const int rc = tiny_prepare(d, a, W, nc);
  if (rc != FAM_OK) return rc;
  const int64_t last = 2LL * a.L * a.T;
  FAM_REQUIRE(phase_begin >= 0 && phase_begin <= phase_end && phase_end <= last + 1, FAM_ERR_INVALID_ARG,
              "fam_tiny_expert: phases [%lld, %lld) outside [0, %lld]", (long long)phase_begin, (long long)phase_end,
              (long long)(last + 1));
  if (phase_begin == phase_end) return FAM_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool two = nc > 16;
  switch (W) {
    case 32: return two ? fam::launch_tiny<32, 2>(a, phase_begin, phase_end, st) : fam::launch_tiny<32, 1>(a, phase_begin, phase_end, st);
    case 64: return two ? fam::launch_tiny<64, 2>(a, phase_begin, phase_end, st) : fam::launch_tiny<64, 1>(a, phase_begin, phase_end, st);
    default: return two ? fam::launch_tiny<128, 2>(a, phase_begin, phase_end, st) : fam::launch_tiny<128, 1>(a, phase_begin, phase_end, st);
  }
}

extern "C" int fam_tiny_context(const fam_tiny_desc* d, void* stream) {
  fam::TinyArgs a;
  int64_t W = 0, nc = 0;
  const int rc = tiny_prepare(d, a, W, nc);
  if (rc != FAM_OK) return rc;
  if (W <= 32) return FAM_OK;
  FAM_LAUNCH(fam::tiny_ctx_rs_kernel, dim3((a.Lcp + 255) / 256, a.L), dim3(256), 0, (hipStream_t)stream, a);
  return fam_host::check_launch("fam_tiny_context");
}
