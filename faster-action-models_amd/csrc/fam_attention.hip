// Flash-style attention on bf16 MFMA (gfx950):  o = softmax(q k^T * scale + mask) v.
//
// Formulation (every kernel).  Scores are computed transposed, S^T = K Q^T, with the key
// tile as the MFMA A-operand and the query tile as the B-operand (v_mfma_f32_16x16x32_bf16).
// A lane then owns ONE query (column l%16) and four keys per 16-key sub-tile, so the running
// max / sum of the online softmax are per-lane scalars reduced over the 4 lane groups with
// two shuffles, and the probabilities already sit in the B-operand layout of the second
// product O^T = V^T P^T (A-operand = V^T read from a transposed LDS tile).  The key order
// inside an MFMA k-block is permuted consistently on both operands (keys {4g..4g+3} and
// {16+4g..16+4g+3} for lane group g), which leaves the dot products unchanged.
//
// attn_short_kernel (Sq <= 64: 32 action tokens over their own 32 keys, over a 1560-token
// context, or over a cached video prefix): one workgroup per (batch, head) holds every
// query; its waves split the keys into contiguous runs of 32-key blocks, each wave with a
// private transposed V tile in LDS and the next block's K/V loads in flight while it
// computes the current one.  The per-wave partial softmax states are merged through LDS in
// wave order at the end (deterministic, no cross-workgroup traffic).
//
// attn_tiled_kernel (Sq > 64: video tokens): a workgroup of 4 waves owns 64 queries of one
// (batch, head); 32-key K/V blocks are staged through LDS and shared by the waves.
//
// Head dims 64 and 128 take specialised kernels first (launch_dh): attn_self_kernel (the action
// tokens over their own keys), attn_small_kernel (up to 128 queries over up to 256 keys),
// attn_cross_kernel (up to 32 queries over a long context, key splits + attn_combine_kernel)
// and attn_long_kernel (128 queries per workgroup over one long key segment); the two kernels
// above take what none of them covers.
//
// Algorithmic bytes per launch: 2*B*H*Dh*(2*Sq + 2*Sk) (+ mask); flops 4*B*H*Sq*Sk*Dh.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "fam_common.h"

namespace fam {

constexpr int KB = 32;  // keys per block
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const bf16* q; int64_t q_bs, q_rs, q_hs;
  const bf16* k0; int64_t k0_bs, k0_rs, k0_hs;
  const bf16* v0; int64_t v0_bs, v0_rs, v0_hs;
  const bf16* k1; int64_t k1_bs, k1_rs, k1_hs;
  const bf16* v1; int64_t v1_bs, v1_rs, v1_hs;
  bf16* o; int64_t o_bs, o_rs, o_hs;
  int64_t H, Sq, sk0, Sk;
  float scale_log2;
  const void* mask; int mask_kind; int64_t mbs, mhs, mqs;
  int splits; float* part_o; float* part_ml;   // key splits over workgroups (grid.y)
  // on-load RMSNorm (+ RoPE) of q / k from the producer's per-16-column sums of squares
  const float* qss; const float* kss; int64_t ssrs, ssbr, qg0, kg0, nwidth;
  const bf16* qnw; const bf16* knw; float neps;
  const float* rcs; const float* rsn; int64_t rrs;
};

// Reciprocal RMS of producer row `row` over the groups [g0, g0 + nwidth/16): the four lane
// groups of a row each sum a quarter (16 groups per chunk of four 16-byte loads) and
// group4_sum adds the quarters in a fixed order.  `first` holds the first chunk, loaded with
// the kernel's other operands.
__device__ __forceinline__ void ss_load(const AttnArgs& a, const float* ss, int64_t row, int64_t g0, int lg,
                                        f32x4 (&r)[4]) {
  const float* p = ss + row * a.ssrs + g0 + lg * (a.nwidth / 64);
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = *reinterpret_cast<const f32x4*>(p + 4 * j);
}
__device__ __forceinline__ float ss_rstd(const AttnArgs& a, const float* ss, int64_t row, int64_t g0, int lg,
                                         const f32x4 (&first)[4]) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) s += (first[j][0] + first[j][1]) + (first[j][2] + first[j][3]);
  const int64_t per = a.nwidth / 64;  // groups per lane group
  for (int64_t c = 16; c < per; c += 16) {
    const float* p = ss + row * a.ssrs + g0 + lg * per + c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + 4 * j);
      s += (v[0] + v[1]) + (v[2] + v[3]);
    }
  }
  s = group4_sum(s);
  return rsqrtf(s / (float)a.nwidth + a.neps);
}
// RMSNorm rounding of the reference (bf16 before the weight) and the RoPE rotation of the
// fragment's four (d, d+1) pairs, in fp32; cs / sn hold the pairs' table entries.
__device__ __forceinline__ bf16x8 norm_rope8(bf16x8 x, float rstd, bf16x8 w, f32x4 cs, f32x4 sn, bool rope) {
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = to_f(to_bf(to_f(to_bf(to_f(x[e]) * rstd)) * to_f(w[e])));
  if (rope) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float x0 = y[2 * p], x1 = y[2 * p + 1];
      y[2 * p] = x0 * cs[p] - x1 * sn[p];
      y[2 * p + 1] = x0 * sn[p] + x1 * cs[p];
    }
  }
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf(y[e]);
  return o;
}

// Row addressing of the two key/value segments of one (batch, head), held in registers:
// key kk < sk0 lives in segment 0, the others in segment 1.  Computing both candidate
// addresses and selecting per lane keeps the loads branch-free.
struct SegRows {
  const bf16* base0; int64_t rs0;
  const bf16* base1; int64_t rs1;
  int64_t sk0;
  __device__ __forceinline__ const bf16* row(int64_t kk) const {
    const bf16* p0 = base0 + kk * rs0;
    const bf16* p1 = base1 + (kk - sk0) * rs1;
    return kk < sk0 ? p0 : p1;
  }
};

__device__ __forceinline__ SegRows key_rows(const AttnArgs& a, int64_t b, int64_t h) {
  SegRows r;
  r.base0 = a.k0 + b * a.k0_bs + h * a.k0_hs; r.rs0 = a.k0_rs;
  r.base1 = a.k1 + b * a.k1_bs + h * a.k1_hs; r.rs1 = a.k1_rs;
  r.sk0 = a.sk0;
  if (a.sk0 == 0) { r.base0 = r.base1; r.rs0 = r.rs1; }   // segment 0 empty: keep both valid
  if (a.Sk == a.sk0) { r.base1 = r.base0; r.rs1 = r.rs0; } // segment 1 empty
  return r;
}
__device__ __forceinline__ SegRows val_rows(const AttnArgs& a, int64_t b, int64_t h) {
  SegRows r;
  r.base0 = a.v0 + b * a.v0_bs + h * a.v0_hs; r.rs0 = a.v0_rs;
  r.base1 = a.v1 + b * a.v1_bs + h * a.v1_hs; r.rs1 = a.v1_rs;
  r.sk0 = a.sk0;
  if (a.sk0 == 0) { r.base0 = r.base1; r.rs0 = r.rs1; }
  if (a.Sk == a.sk0) { r.base1 = r.base0; r.rs1 = r.rs0; }
  return r;
}

// scaled (log2 domain) and masked score of query qi and key kk; branch-free per lane (the
// mask kind is uniform): out-of-range queries/keys read a clamped mask element
__device__ __forceinline__ float score(const AttnArgs& a, float raw, int64_t b, int64_t h, int64_t qi, bool qvalid,
                                       int64_t kk) {
  const bool kvalid = kk < a.Sk;
  float v = raw * a.scale_log2;
  if (a.mask_kind != FAM_MASK_NONE) {
    const int64_t mi = b * a.mbs + h * a.mhs + (qvalid ? qi : 0) * a.mqs + (kvalid ? kk : 0);
    if (a.mask_kind == FAM_MASK_BOOL) {
      v = reinterpret_cast<const uint8_t*>(a.mask)[mi] ? v : -INFINITY;
    } else if (a.mask_kind == FAM_MASK_ADD_F32) {
      v += reinterpret_cast<const float*>(a.mask)[mi] * kLog2e;
    } else {
      v += to_f(reinterpret_cast<const bf16*>(a.mask)[mi]) * kLog2e;
    }
  }
  return kvalid ? v : -INFINITY;
}

// Online-softmax update of one query column with the 8 scores of a 32-key block; returns
// the probabilities as the bf16 B-operand of the P V product and rescales the accumulator.
template <int NDT>
__device__ __forceinline__ bf16x8 softmax_update(const float (&s)[2][4], float& m_run, float& l_run, f32x4 (&oacc)[NDT]) {
  float mloc = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) mloc = fmaxf(mloc, s[kt][e]);
  const float m_new = fmaxf(m_run, group4_max(mloc));
  bf16x8 pf;
  if (m_new == -INFINITY) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pf[j] = (bf16)0.0f;
    return pf;
  }
  const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run = -inf -> 0
  float psum = 0.f;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __builtin_amdgcn_exp2f(s[kt][e] - m_new);
      psum += p;
      pf[kt * 4 + e] = to_bf(p);
    }
  l_run = l_run * alpha + group4_sum(psum);
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] *= alpha;
  m_run = m_new;
  return pf;
}

// ---------------------------------------------------------------------------------------
template <int DH, int QT, int NW, bool QN = false, bool KN = false>
__global__ __launch_bounds__(NW * 64) void attn_short_kernel(AttnArgs a) {
  constexpr int NC = (DH + 31) / 32;   // 32-wide k-chunks of the head dim (zero padded)
  constexpr int NDT = (DH + 15) / 16;  // 16-row output tiles of the head dim
  constexpr int VROWS = NDT * 16;
  constexpr int NVC = (KB * DH / 8 + 63) / 64;  // 16-byte V chunks per lane per block
  constexpr int NQ = QT * 16;
  __shared__ bf16 Vt[NW][VROWS][KB + 8];
  __shared__ float s_m[NW][NQ], s_l[NW][NQ];
  __shared__ float s_o[NQ][DH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const uint32_t bh32 = blockIdx.x, H32 = (uint32_t)a.H;
  const int64_t bh = bh32, b = bh32 / H32, h = bh32 - (uint32_t)b * H32;
  // this workgroup's key blocks (split blockIdx.y of a.splits), divided among its waves
  const int64_t nkb_all = (a.Sk + KB - 1) / KB;
  const int64_t per_split = (nkb_all + a.splits - 1) / a.splits;
  const int64_t wg_beg = std::min(nkb_all, (int64_t)blockIdx.y * per_split);
  const int64_t wg_end = std::min(nkb_all, wg_beg + per_split);
  const int64_t per = (wg_end - wg_beg + NW - 1) / NW;
  const int64_t kb_beg = std::min(wg_end, wg_beg + (int64_t)wave * per), kb_end = std::min(wg_end, kb_beg + per);

  const SegRows krows = key_rows(a, b, h), vrows = val_rows(a, b, h);
  const int64_t Sk = a.Sk;
  const bf16* ksafe = krows.row(0);
  const bf16* vsafe = vrows.row(0);
  // Raw loads of one key block from clamped addresses (no selects between the loads).  A key
  // past Sk reads row 0: its score is masked to -inf below and its V row is weighted by 0.
  // k normalisation operands of one block (KN): sums-of-squares chunk and RoPE entries per key row
  struct KNorm {
    f32x4 ss[2][4];
    f32x4 cs[2][NC], sn[2][NC];
  };
  const bool rope = a.rcs != nullptr;
  const float* rsafe = rope ? a.rcs : a.kss ? a.kss : a.qss;
  auto kn_load = [&](int64_t blk, KNorm& n) {
    if constexpr (KN) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int64_t kk = blk * KB + kt * 16 + l16;
        const int64_t kc = kk < a.Sk ? kk : 0;
        ss_load(a, a.kss, b * a.ssbr + kc, a.kg0, lg, n.ss[kt]);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int64_t t = kc * a.rrs + (c * 32 + lg * 8) / 2;
          n.cs[kt][c] = *reinterpret_cast<const f32x4*>(rope ? a.rcs + t : rsafe);
          n.sn[kt][c] = *reinterpret_cast<const f32x4*>(rope ? a.rsn + t : rsafe);
        }
      }
    }
  };
  bf16x8 knw[NC];
  if constexpr (KN) {
#pragma unroll
    for (int c = 0; c < NC; ++c) knw[c] = load8(a.knw + h * DH + c * 32 + lg * 8);
  }

  auto gload = [&](int64_t blk, bf16x8 (&kf)[2][NC], bf16x8 (&vc)[NVC]) {
    const int64_t kb = blk * KB;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t kk = kb + kt * 16 + l16;
        const int d0 = c * 32 + lg * 8;
        const bool ok = kk < Sk && d0 < DH;
        kf[kt][c] = load8(ok ? krows.row(kk) + d0 : ksafe);
      }
#pragma unroll
    for (int p = 0; p < NVC; ++p) {
      const int cidx = lane + 64 * p;
      const int key = cidx / (DH / 8), d0 = (cidx % (DH / 8)) * 8;
      const int64_t kk = kb + key;
      const bool ok = cidx < KB * DH / 8 && kk < Sk;
      vc[p] = load8(ok ? vrows.row(kk) + d0 : vsafe);
    }
  };

  bf16x8 qf[QT][NC];
  const bf16* qbase = a.q + b * a.q_bs + h * a.q_hs;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t qi = qt * 16 + l16;
      const int d0 = c * 32 + lg * 8;
      qf[qt][c] = load8(qi < a.Sq && d0 < DH ? qbase + qi * a.q_rs + d0 : qbase);
    }
  // q normalisation operands (QN): sums of squares, weights, RoPE entries of the lane's rows
  f32x4 qss[QT][4], qcs[QT][NC], qsn[QT][NC];
  bf16x8 qnw[NC];
  if constexpr (QN) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int64_t qi = qt * 16 + l16;
      const int64_t qc = qi < a.Sq ? qi : 0;
      ss_load(a, a.qss, b * a.ssbr + qc, a.qg0, lg, qss[qt]);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t t = qc * a.rrs + (c * 32 + lg * 8) / 2;
        qcs[qt][c] = *reinterpret_cast<const f32x4*>(rope ? a.rcs + t : rsafe);
        qsn[qt][c] = *reinterpret_cast<const f32x4*>(rope ? a.rsn + t : rsafe);
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) qnw[c] = load8(a.qnw + h * DH + c * 32 + lg * 8);
  }
  bf16x8 kA[2][NC], vA[NVC], kB[2][NC], vB[NVC];
  KNorm nA, nB;
  if (kb_beg < kb_end) {
    gload(kb_beg, kA, vA);
    kn_load(kb_beg, nA);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (QN) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int64_t qi = qt * 16 + l16;
      const float r = ss_rstd(a, a.qss, b * a.ssbr + (qi < a.Sq ? qi : 0), a.qg0, lg, qss[qt]);
#pragma unroll
      for (int c = 0; c < NC; ++c) qf[qt][c] = norm_rope8(qf[qt][c], r, qnw[c], qcs[qt][c], qsn[qt][c], rope);
    }
  }
  if constexpr (DH < 32) {
    // zero-padded head dim: the padding lanes of the q fragments must be exactly 0
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (c * 32 + lg * 8 >= DH) qf[qt][c] = zero8();
  }

  f32x4 oacc[QT][NDT];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int t = 0; t < NDT; ++t) oacc[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // one 32-key block: V -> this wave's transposed LDS tile, S^T = K Q^T, online softmax, O^T += V^T P^T
  auto process = [&](int64_t blk, bf16x8 (&kf)[2][NC], const bf16x8 (&vc)[NVC], const KNorm& kn) {
    const int64_t kb = blk * KB;
    if constexpr (KN) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int64_t kk = kb + kt * 16 + l16;
        const float r = ss_rstd(a, a.kss, b * a.ssbr + (kk < a.Sk ? kk : 0), a.kg0, lg, kn.ss[kt]);
#pragma unroll
        for (int c = 0; c < NC; ++c) kf[kt][c] = norm_rope8(kf[kt][c], r, knw[c], kn.cs[kt][c], kn.sn[kt][c], rope);
      }
    }
    if constexpr (DH < 32) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int c = 0; c < NC; ++c)
          if (c * 32 + lg * 8 >= DH) kf[kt][c] = zero8();
    }
#pragma unroll
    for (int p = 0; p < NVC; ++p) {
      const int cidx = lane + 64 * p;
      if (cidx < KB * DH / 8) {
        const int key = cidx / (DH / 8), d0 = (cidx % (DH / 8)) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) Vt[wave][d0 + e][key] = vc[p][e];
      }
    }
    __builtin_amdgcn_wave_barrier();
    bf16x8 vfr[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const int d = t * 16 + l16;
      if (d < DH) {
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(&Vt[wave][d][lg * 4]);
        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(&Vt[wave][d][16 + lg * 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) { vfr[t][e] = lo[e]; vfr[t][4 + e] = hi[e]; }
      } else {
        vfr[t] = zero8();
      }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int64_t qi = qt * 16 + l16;
      const bool qvalid = qi < a.Sq;
      float sc[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) sacc = mfma16(kf[kt][c], qf[qt][c], sacc);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[kt][e] = score(a, sacc[e], b, h, qi, qvalid, kb + kt * 16 + lg * 4 + e);
      }
      const bf16x8 pf = softmax_update<NDT>(sc, m_run[qt], l_run[qt], oacc[qt]);
#pragma unroll
      for (int t = 0; t < NDT; ++t) oacc[qt][t] = mfma16(vfr[t], pf, oacc[qt][t]);
    }
    __builtin_amdgcn_wave_barrier();  // the next block may overwrite this wave's V tile
  };

  // two register sets: the next block's loads are in flight while the current one computes
  for (int64_t blk = kb_beg; blk < kb_end; blk += 2) {
    if (blk + 1 < kb_end) {
      gload(blk + 1, kB, vB);
      kn_load(blk + 1, nB);
    }
    __builtin_amdgcn_sched_barrier(0);
    process(blk, kA, vA, nA);
    if (blk + 1 >= kb_end) break;
    if (blk + 2 < kb_end) {
      gload(blk + 2, kA, vA);
      kn_load(blk + 2, nA);
    }
    __builtin_amdgcn_sched_barrier(0);
    process(blk + 1, kB, vB, nB);
  }

  // ---- merge the waves' partial states in wave order
  if constexpr (NW == 1) {
    // one wave: its accumulator is the result; lanes with lg == 0 hold (m, l) of query l16
    (void)s_m; (void)s_l;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int64_t q = qt * 16 + l16;
      if (q >= a.Sq) continue;
      const float L = l_run[qt];
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const int d0 = t * 16 + lg * 4;
        if (d0 >= DH) continue;
        const f32x4 v = oacc[qt][t];
        if (a.splits > 1) {
          const int64_t row = ((int64_t)blockIdx.y * gridDim.x + bh) * a.Sq + q;
          *reinterpret_cast<f32x4*>(a.part_o + row * DH + d0) = v;
          if (d0 == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = make_float2(m_run[qt], L);
        } else {
          const float inv = L > 0.f ? 1.0f / L : 0.f;
          bf16x4 ov;
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[e] = to_bf(v[e] * inv);
          *reinterpret_cast<bf16x4*>(a.o + b * a.o_bs + q * a.o_rs + h * a.o_hs + d0) = ov;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
    if (lg == 0) { s_m[wave][qt * 16 + l16] = m_run[qt]; s_l[wave][qt * 16 + l16] = l_run[qt]; }
  __syncthreads();
  float wscale[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = qt * 16 + l16;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_m[w][q]);
    wscale[qt] = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[qt] - mx);
  }
  for (int w = 0; w < NW; ++w) {
    if (wave == w) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const int d0 = t * 16 + lg * 4;
          if (d0 < DH) {
            f32x4* dst = reinterpret_cast<f32x4*>(&s_o[qt * 16 + l16][d0]);
            const f32x4 v = oacc[qt][t] * wscale[qt];
            *dst = (w == 0) ? v : (*dst + v);
          }
        }
    }
    __syncthreads();
  }
  for (int idx = tid; idx < NQ * (DH / 4); idx += NW * 64) {
    const int q = idx / (DH / 4), d0 = (idx % (DH / 4)) * 4;
    if (q >= a.Sq) continue;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_m[w][q]);
    float L = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) L += s_l[w][q] * __builtin_amdgcn_exp2f(s_m[w][q] - mx);
    }
    const f32x4 v = *reinterpret_cast<const f32x4*>(&s_o[q][d0]);
    if (a.splits > 1) {
      // unnormalised partial of this split, merged by fam_attention_combine
      const int64_t row = ((int64_t)blockIdx.y * gridDim.x + bh) * a.Sq + q;
      *reinterpret_cast<f32x4*>(a.part_o + row * DH + d0) = v;
      if (d0 == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = make_float2(mx, L);
      continue;
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    bf16x4 ov;
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = to_bf(v[e] * inv);
    *reinterpret_cast<bf16x4*>(a.o + b * a.o_bs + q * a.o_rs + h * a.o_hs + d0) = ov;
  }
}

// ---------------------------------------------------------------------------------------
// attn_self_kernel: the action tokens' own attention (Sq <= 32, Sk <= 32, one key segment, no
// mask), one workgroup of 4 waves per (batch, head).  All 256 threads stage the head's q and k
// (normalised and rotated on the way when QKN) and the transposed V in LDS, one 16-byte chunk
// of each per thread (two for Dh = 128); then waves 0 and 1 each finish 16 queries over the
// (single) key block with exact softmax, no running rescale and no merge.
template <int DH, bool QKN>
__global__ __launch_bounds__(256) void attn_self_kernel(AttnArgs a) {
  constexpr int NC = DH / 32;             // 32-wide k-chunks of the head dim
  constexpr int NDT = DH / 16;            // 16-row output tiles of the head dim
  constexpr int CPR = DH / 8;             // 16-byte chunks per row
  constexpr int CH = 32 * CPR / 256;      // chunks per thread per tensor (1 or 2)
  constexpr int LD = DH + 8;              // padded LDS rows (bf16)
  __shared__ bf16 Qs[32][LD];
  __shared__ bf16 Ks[32][LD];
  // V row-major ([key][dim], pitch DH + 16), read back as V^T by transposing LDS reads
  __shared__ __attribute__((aligned(16))) bf16 Vs[32][DH + 16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const uint32_t bh = blockIdx.x, H32 = (uint32_t)a.H;
  const uint32_t b = bh / H32, h = bh - b * H32;
  const int Sq = (int)a.Sq, Sk = (int)a.Sk;
  const bf16* qb = a.q + b * a.q_bs + h * a.q_hs;
  const bf16* kb = a.k0 + b * a.k0_bs + h * a.k0_hs;
  const bf16* vb = a.v0 + b * a.v0_bs + h * a.v0_hs;

  // ---- phase 1: raw loads of this thread's chunks (row r, dims d0..d0+7)
  bf16x8 qr[CH], kr[CH], vr[CH];
  f32x4 qss[CH][2], kss[CH][2], qcs[CH], qsn[CH], kcs[CH], ksn[CH];
  bf16x8 qw[CH], kw[CH];
  const bool rope = QKN && a.rcs != nullptr;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = tid + 256 * c, r = idx / CPR, d0 = (idx % CPR) * 8;
    const int rq = r < Sq ? r : 0, rk = r < Sk ? r : 0;
    qr[c] = load8(qb + rq * a.q_rs + d0);
    kr[c] = load8(kb + rk * a.k0_rs + d0);
    vr[c] = load8(vb + rk * a.v0_rs + d0);
    if constexpr (QKN) {
      // the row's sums of squares: CPR threads share a row, each sums nwidth/16/CPR groups
      const int64_t per = a.nwidth / 16 / CPR;
      const float* qsp = a.qss + (b * a.ssbr + rq) * a.ssrs + a.qg0 + (idx % CPR) * per;
      const float* ksp = a.kss + (b * a.ssbr + rk) * a.ssrs + a.kg0 + (idx % CPR) * per;
      // (a share of 4 groups reads its first 16 bytes twice and counts them once, below)
      qss[c][0] = *reinterpret_cast<const f32x4*>(qsp);
      qss[c][1] = *reinterpret_cast<const f32x4*>(per >= 8 ? qsp + 4 : qsp);
      kss[c][0] = *reinterpret_cast<const f32x4*>(ksp);
      kss[c][1] = *reinterpret_cast<const f32x4*>(per >= 8 ? ksp + 4 : ksp);
      qw[c] = load8(a.qnw + h * DH + d0);
      kw[c] = load8(a.knw + h * DH + d0);
      const float* cb = rope ? a.rcs : a.qss;
      const float* sb = rope ? a.rsn : a.qss;
      qcs[c] = *reinterpret_cast<const f32x4*>(cb + (rope ? rq * a.rrs + d0 / 2 : 0));
      qsn[c] = *reinterpret_cast<const f32x4*>(sb + (rope ? rq * a.rrs + d0 / 2 : 0));
      kcs[c] = *reinterpret_cast<const f32x4*>(cb + (rope ? rk * a.rrs + d0 / 2 : 0));
      ksn[c] = *reinterpret_cast<const f32x4*>(sb + (rope ? rk * a.rrs + d0 / 2 : 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- phase 2: normalise, stage in LDS
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = tid + 256 * c, r = idx / CPR, d0 = (idx % CPR) * 8;
    bf16x8 qn = qr[c], kn = kr[c];
    if constexpr (QKN) {
      const int64_t per = a.nwidth / 16 / CPR;
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j == 1 && per < 8) break;
        sq += (qss[c][j][0] + qss[c][j][1]) + (qss[c][j][2] + qss[c][j][3]);
        sk += (kss[c][j][0] + kss[c][j][1]) + (kss[c][j][2] + kss[c][j][3]);
      }
      // groups beyond the first 8 of this thread's share (wider rows), in order
      for (int64_t g = 8; g < per; g += 4) {
        const int rq = r < Sq ? r : 0, rk = r < Sk ? r : 0;
        const f32x4 x = *reinterpret_cast<const f32x4*>(a.qss + (b * a.ssbr + rq) * a.ssrs + a.qg0 + (idx % CPR) * per + g);
        const f32x4 y = *reinterpret_cast<const f32x4*>(a.kss + (b * a.ssbr + rk) * a.ssrs + a.kg0 + (idx % CPR) * per + g);
        sq += (x[0] + x[1]) + (x[2] + x[3]);
        sk += (y[0] + y[1]) + (y[2] + y[3]);
      }
      // sum over the CPR threads of the row (consecutive lanes), fixed butterfly order
#pragma unroll
      for (int o = 1; o < CPR; o <<= 1) {
        sq += __shfl_xor(sq, o, kWave);
        sk += __shfl_xor(sk, o, kWave);
      }
      const float rq = rsqrtf(sq / (float)a.nwidth + a.neps), rk = rsqrtf(sk / (float)a.nwidth + a.neps);
      qn = norm_rope8(qr[c], rq, qw[c], qcs[c], qsn[c], rope);
      kn = norm_rope8(kr[c], rk, kw[c], kcs[c], ksn[c], rope);
    }
    *reinterpret_cast<bf16x8*>(&Qs[r][d0]) = qn;
    *reinterpret_cast<bf16x8*>(&Ks[r][d0]) = kn;
    *reinterpret_cast<bf16x8*>(&Vs[r][d0]) = vr[c];
  }
  __syncthreads();
  if (wave >= 2 || wave * 16 >= Sq) return;

  // ---- phase 3: wave w finishes queries 16w..16w+15 (S^T = K Q^T, lane = one query)
  const int qt = wave;
  bf16x8 qf[NC], kf[2][NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    qf[c] = *reinterpret_cast<const bf16x8*>(&Qs[qt * 16 + l16][c * 32 + lg * 8]);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) kf[kt][c] = *reinterpret_cast<const bf16x8*>(&Ks[kt * 16 + l16][c * 32 + lg * 8]);
  }
  float sc[2][4];
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) acc = mfma16(kf[kt][c], qf[c], acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int kk = kt * 16 + lg * 4 + e;   // keys {4g..4g+3} and {16+4g..16+4g+3} of lane group g
      const float v = kk < Sk ? acc[e] * a.scale_log2 : -INFINITY;
      sc[kt][e] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = group4_max(mx);
  float psum = 0.f;
  bf16x8 pf;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pv = __builtin_amdgcn_exp2f(sc[kt][e] - mx);
      psum += pv;
      pf[kt * 4 + e] = to_bf(pv);
    }
  const float inv = 1.0f / group4_sum(psum);
  const int q = qt * 16 + l16;
  // V^T fragment of dim tile t: lane s of a 16-lane group loads key 4 lg + s / 4 (+ 16), dims
  // 16 t + 4 (s % 4) .. + 3; lane i receives keys 4 lg .. 4 lg + 3 of dim 16 t + i (P's order)
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    const int key = lg * 4 + (l16 >> 2), dim = t * 16 + 4 * (l16 & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&Vs[key][dim]);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&Vs[key + 16][dim]);
    const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const bf16x8 vf = __builtin_bit_cast(bf16x8, v8);
    const f32x4 o = mfma16(vf, pf, f32x4{0.f, 0.f, 0.f, 0.f});   // O^T[d = 16t + 4lg + i][q]
    if (q < Sq) {
      bf16x4 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = to_bf(o[e] * inv);
      *reinterpret_cast<bf16x4*>(a.o + b * a.o_bs + q * a.o_rs + h * a.o_hs + t * 16 + lg * 4) = ov;
    }
  }
}

// ---------------------------------------------------------------------------------------
// attn_small_kernel: up to 32 queries over up to 32 NW keys (two segments, optional mask): the
// MoT joint attention of the action tokens over [cached video K/V ; action K/V] and their
// cross-attention to a short context; without on-load q normalisation also up to 128 queries
// as chunks of 32 (grid.z: the video prefill's 98 tokens over their own 98 keys or 129 text
// keys).  Grid (batch * head, NV, chunks): workgroup (bh, y, z) produces output dims
// [y DH/NV, (y+1) DH/NV) of queries [32 z, 32 z + 32) of its head, one wave per 32-key block.  Every workgroup of
// a head computes the same full scores, so the dim split needs no combine; it divides the V
// reads and spreads a head over NV CUs.  Every global load is issued before the first use:
//   - the queries, once per workgroup, staged in LDS (NSS > 0: q arrives raw from
//     fam_gemm_final and is RMS-normalised on the way from the producer's per-16-column sums of
//     squares, the DH/8 threads of a query each summing a share of the row);
//   - the wave's K block as MFMA A-fragments straight from global memory;
//   - the wave's V block (its dims only), row-major into the wave's own LDS rows, read back
//     as the V^T operand through transposing LDS reads;
//   - the mask entries of the lane's scores.
// Keys past Sk are not loaded.  Each wave takes an exact softmax over its block (S^T = K Q^T, a
// lane holds one query); the waves' (m, l, o) are merged through LDS in wave order.
// MK: the mask's kind as a template constant (0 none, 1 bool, 2 additive fp32 / bf16), so that
// each instantiation has one load path (a runtime switch merges the paths' pending loads and
// the compiler then waits for all of them in every path)
template <int DH, int NW, int NV, int NSS, int MK>
__global__ __launch_bounds__(NW * 64) void attn_small_kernel(AttnArgs a) {
  constexpr int NC = DH / 32, CPR = DH / 8, NT = NW * 64;
  constexpr int DVW = DH / NV, NDT = DVW / 16, VCPR = DVW / 8;   // this workgroup's output dims
  constexpr int NVC = KB * VCPR / 64;                              // 16-byte V chunks per lane
  constexpr int VLD = DVW + 16;      // V row pitch: 8 rows x 32 bytes of a transposing read
                                     // land in distinct banks
  constexpr int QLD = DH + 8;
  constexpr int QCH = (32 * CPR + NT - 1) / NT;                    // q chunks per thread
  constexpr int VS_BYTES = NW * KB * VLD * 2, SO_BYTES = NW * 32 * DVW * 4;
  constexpr int LDS_BYTES = VS_BYTES > SO_BYTES ? VS_BYTES : SO_BYTES;
  constexpr bool QN = NSS > 0;
  static_assert(NVC >= 1 && NDT >= 1, "unsupported dim split");
  // the V blocks, then (after a barrier) the waves' fp32 partial outputs, in one buffer
  __shared__ __attribute__((aligned(16))) unsigned char smem[LDS_BYTES];
  __shared__ __attribute__((aligned(16))) bf16 Qs[32][QLD];
  __shared__ float s_m[NW][32], s_l[NW][32];
  bf16 (*Vs)[KB][VLD] = reinterpret_cast<bf16 (*)[KB][VLD]>(smem);
  float (*So)[32][DVW] = reinterpret_cast<float (*)[32][DVW]>(smem);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const uint32_t bh32 = blockIdx.x, H32 = (uint32_t)a.H;
  const int64_t b = bh32 / H32, h = bh32 - (uint32_t)b * H32;
  const int dv0 = (int)blockIdx.y * DVW;
  // grid.z: chunks of 32 queries (more than 32 queries without on-load normalisation); Sq is
  // this chunk's query count, qz its first query
  const int qz = (int)blockIdx.z * 32;
  const int Sq = min(32, (int)a.Sq - qz), Sk = (int)a.Sk;
  const int k0 = wave * KB;
  const SegRows krows = key_rows(a, b, h), vrows = val_rows(a, b, h);

  // ---- phase 1: every load
  const bf16* qbase = a.q + b * a.q_bs + h * a.q_hs + (int64_t)qz * a.q_rs;
  bf16x8 qr[QCH], qw[QCH];
  f32x4 ssv[QCH][QN ? NSS : 1];
  const int nss = QN ? (int)(a.nwidth / 16 / CPR / 4) : 0;   // 16-byte chunks of a thread's share
#pragma unroll
  for (int j = 0; j < QCH; ++j) {
    const int idx = tid + NT * j, q = idx / CPR, d0 = (idx % CPR) * 8;
    const int qc = q < Sq ? q : 0;
    qr[j] = load8(qbase + qc * a.q_rs + d0);
    if constexpr (QN) {
      qw[j] = load8(a.qnw + h * DH + d0);
      const float* p = a.qss + (b * a.ssbr + qz + qc) * a.ssrs + a.qg0 + (idx % CPR) * (a.nwidth / 16 / CPR);
#pragma unroll
      for (int u = 0; u < NSS; ++u) ssv[j][u] = *reinterpret_cast<const f32x4*>(p + 4 * (u < nss ? u : 0));
    }
  }
  // K, V and mask loads are unconditional (keys past Sk read key 0 and are zeroed or masked
  // after the wait) and keep raw bits until then: a load under a branch, consumed on the spot,
  // made the compiler wait for every load issued before it, one round trip per load
  bf16x8 kf[2][NC];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int kk = k0 + kt * 16 + l16;
    const bf16* kr = krows.row(kk < Sk ? kk : 0);
#pragma unroll
    for (int c = 0; c < NC; ++c) kf[kt][c] = load8(kr + c * 32 + lg * 8);
  }
  bf16x8 vc[NVC];
#pragma unroll
  for (int p = 0; p < NVC; ++p) {
    const int cidx = lane + 64 * p, key = cidx / VCPR, d0 = dv0 + (cidx % VCPR) * 8;
    const int kk = k0 + key;
    vc[p] = load8(vrows.row(kk < Sk ? kk : 0) + d0);
  }
  // the lane's mask entries, raw: buffer loads off the (batch, head) base with 32-bit offsets
  // (64-bit addresses for 16 entries cost enough registers to force a wait mid-issue)
  uint32_t mraw[2][2][4];
  const int mk = a.mask_kind;
  if constexpr (MK == 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) mraw[t][kt][e] = 0u;
  } else {
    const int msz = MK == 1 ? 1 : (mk == FAM_MASK_ADD_F32 ? 4 : 2);
    const auto mrs = buffer_rsrc((const void*)((const char*)a.mask + (b * a.mbs + h * a.mhs + (int64_t)qz * a.mqs) * msz),
                                 (uint32_t)(((int64_t)(Sq - 1) * a.mqs + Sk) * msz));
    auto moff = [&](int t, int kt, int e) {
      const int q = t * 16 + l16, kk = k0 + kt * 16 + lg * 4 + e;
      return ((uint32_t)(q < Sq ? q : 0) * (uint32_t)a.mqs + (uint32_t)(kk < Sk ? kk : 0)) * (uint32_t)msz;
    };
    if constexpr (MK == 1) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) mraw[t][kt][e] = __builtin_amdgcn_raw_buffer_load_b8(mrs, moff(t, kt, e), 0, 0);
    } else if (mk == FAM_MASK_ADD_F32) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) mraw[t][kt][e] = __builtin_amdgcn_raw_buffer_load_b32(mrs, moff(t, kt, e), 0, 0);
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) mraw[t][kt][e] = __builtin_amdgcn_raw_buffer_load_b16(mrs, moff(t, kt, e), 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // keys past Sk: zero K and V fragments; the mask entries as additive log2-domain terms
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (k0 + kt * 16 + l16 >= Sk) kf[kt][c] = zero8();
#pragma unroll
  for (int p = 0; p < NVC; ++p)
    if (k0 + (lane + 64 * p) / VCPR >= Sk) vc[p] = zero8();
  float madd[2][2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t r = mraw[t][kt][e];
        float m = 0.f;
        if constexpr (MK == 1) m = r ? 0.f : -INFINITY;
        else if constexpr (MK == 2) m = (mk == FAM_MASK_ADD_F32 ? __uint_as_float(r) : __uint_as_float(r << 16)) * kLog2e;
        madd[t][kt][e] = m;
      }

  // ---- phase 2: queries (normalised) and the V block into LDS
#pragma unroll
  for (int j = 0; j < QCH; ++j) {
    const int idx = tid + NT * j, q = idx / CPR, d0 = (idx % CPR) * 8;
    bf16x8 qn = qr[j];
    if constexpr (QN) {
      float sq = 0.f;
#pragma unroll
      for (int u = 0; u < NSS; ++u)
        if (u < nss) sq += (ssv[j][u][0] + ssv[j][u][1]) + (ssv[j][u][2] + ssv[j][u][3]);
      // the CPR threads of a query are consecutive lanes: fixed butterfly order
#pragma unroll
      for (int o = 1; o < CPR; o <<= 1) sq += __shfl_xor(sq, o, kWave);
      const float rstd = rsqrtf(sq / (float)a.nwidth + a.neps);
      const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
      qn = norm_rope8(qr[j], rstd, qw[j], zero4, zero4, false);
    }
    if (q < 32 && idx < 32 * CPR) *reinterpret_cast<bf16x8*>(&Qs[q][d0]) = qn;
  }
#pragma unroll
  for (int p = 0; p < NVC; ++p) {
    const int cidx = lane + 64 * p, key = cidx / VCPR, d0 = (cidx % VCPR) * 8;
    *reinterpret_cast<bf16x8*>(&Vs[wave][key][d0]) = vc[p];
  }
  __syncthreads();

  // ---- the block's scores and exact softmax, per query tile (a lane holds query t*16 + l16)
  float mw[2], lw[2];
  bf16x8 pf[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    bf16x8 qf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const bf16x8*>(&Qs[t * 16 + l16][c * 32 + lg * 8]);
    float sc[2][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) acc = mfma16(kf[kt][c], qf[c], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = k0 + kt * 16 + lg * 4 + e;
        const float v = kk < Sk ? acc[e] * a.scale_log2 + madd[t][kt][e] : -INFINITY;
        sc[kt][e] = v;
        mloc = fmaxf(mloc, v);
      }
    }
    const float m = group4_max(mloc);
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pv = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc[kt][e] - m);
        psum += pv;
        pf[t][kt * 4 + e] = to_bf(pv);
      }
    mw[t] = m;
    lw[t] = group4_sum(psum);
  }
  // O^T of the block over this workgroup's dims: V^T (row = dim, k = key in the score order
  // above) from the row-major V rows with transposing reads -- lane s of a 16-lane group loads
  // key 4lg + s/4 (+16 for the upper half), dims 16dt + 4(s%4) .. +3, and lane i receives keys
  // 4lg .. 4lg+3 of dim 16dt + i
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  f32x4 oacc[2][NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int key = lg * 4 + (l16 >> 2), dim = dt * 16 + 4 * (l16 & 3);
    lds_s16x4* p0 = (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&Vs[wave][key][dim];
    lds_s16x4* p1 = (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&Vs[wave][key + 16][dim];
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1);
    const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const bf16x8 vf = __builtin_bit_cast(bf16x8, v8);
#pragma unroll
    for (int t = 0; t < 2; ++t) oacc[t][dt] = mfma16(vf, pf[t], f32x4{0.f, 0.f, 0.f, 0.f});
  }

  // ---- phase 3: merge the waves' blocks in wave order
  __syncthreads();   // every V read is done: the partial outputs reuse the buffer
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int q = t * 16 + l16;
    if (lg == 0) { s_m[wave][q] = mw[t]; s_l[wave][q] = lw[t]; }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<f32x4*>(&So[wave][q][dt * 16 + lg * 4]) = oacc[t][dt];
  }
  __syncthreads();
  for (int idx = tid; idx < Sq * (DVW / 4); idx += NT) {
    const int q = idx / (DVW / 4), d0 = (idx % (DVW / 4)) * 4;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_m[w][q]);
    float L = 0.f;
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float sw = __builtin_amdgcn_exp2f(s_m[w][q] - mx);   // an empty block: -inf -> 0
        L += s_l[w][q] * sw;
        o += *reinterpret_cast<const f32x4*>(&So[w][q][d0]) * sw;
      }
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    bf16x4 ov;
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = to_bf(o[e] * inv);
    *reinterpret_cast<bf16x4*>(a.o + b * a.o_bs + (int64_t)(qz + q) * a.o_rs + h * a.o_hs + dv0 + d0) = ov;
  }
}

// ---------------------------------------------------------------------------------------
// attn_cross_kernel: 32 or fewer queries over a long key sequence in one segment, no mask (the
// action tokens over the context).  Grid (batch*head, key split), 4 waves.  The workgroup's
// threads normalise the head's queries once into LDS (QN: RMSNorm from the producer's sums of
// squares); each wave then streams its own run of 32-key blocks with the next block's loads
// in flight, and the four partial softmax states are merged through LDS with two barriers.
// Output: o, or with splits the unnormalised partial (o, m, l) merged by attn_combine_kernel.
template <int DH, bool QN>
__global__ __launch_bounds__(256) void attn_cross_kernel(AttnArgs a) {
  constexpr int NW = 4;
  constexpr int NC = DH / 32, NDT = DH / 16, CPR = DH / 8, CH = 32 * CPR / 256;
  constexpr int NVC = KB * DH / 8 / 64;    // 16-byte V chunks per lane per block
  constexpr int LD = DH + 8;
  __shared__ bf16 Qs[32][LD];
  // each wave's V block row-major ([key][dim], pitch DH + 16: 8 rows x 32 bytes of a
  // transposing read land in distinct banks), read back as V^T by ds_read_b64_tr_b16
  constexpr int VLD = DH + 16;
  __shared__ __attribute__((aligned(16))) bf16 Vs[NW][KB][VLD];
  __shared__ float s_m[NW][32], s_l[NW][32];
  __shared__ float s_o[NW][32][DH + 4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const uint32_t bh = blockIdx.x, H32 = (uint32_t)a.H;
  const uint32_t b = bh / H32, h = bh - b * H32;
  const int Sq = (int)a.Sq, Sk = (int)a.Sk;
  const int nkb_all = (Sk + KB - 1) / KB;
  const int per_split = (nkb_all + a.splits - 1) / a.splits;
  const int wg_beg = min(nkb_all, (int)blockIdx.y * per_split);
  const int wg_end = min(nkb_all, wg_beg + per_split);
  const int per = (wg_end - wg_beg + NW - 1) / NW;
  const int kb_beg = min(wg_end, wg_beg + wave * per), kb_end = min(wg_end, kb_beg + per);

  const bf16* qb = a.q + b * a.q_bs + h * a.q_hs;
  const bf16* kbase = a.k0 + b * a.k0_bs + h * a.k0_hs;
  const bf16* vbase = a.v0 + b * a.v0_bs + h * a.v0_hs;
  auto gload = [&](int blk, bf16x8 (&kf)[2][NC], bf16x8 (&vc)[NVC]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int kk = blk * KB + kt * 16 + l16;
#pragma unroll
      for (int c = 0; c < NC; ++c) kf[kt][c] = load8(kbase + (int64_t)(kk < Sk ? kk : 0) * a.k0_rs + c * 32 + lg * 8);
    }
#pragma unroll
    for (int p = 0; p < NVC; ++p) {
      const int cidx = lane + 64 * p, key = cidx / CPR, d0 = (cidx % CPR) * 8;
      const int kk = blk * KB + key;
      vc[p] = load8(vbase + (int64_t)(kk < Sk ? kk : 0) * a.v0_rs + d0);
    }
  };

  // ---- phase 1: raw loads (this thread's query chunks and their norm operands; the wave's first block)
  bf16x8 qr[CH], qw[CH];
  f32x4 qss[CH][2];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = tid + 256 * c, r = idx / CPR, d0 = (idx % CPR) * 8;
    const int rq = r < Sq ? r : 0;
    qr[c] = load8(qb + rq * a.q_rs + d0);
    if constexpr (QN) {
      const int64_t sper = a.nwidth / 16 / CPR;
      const float* qsp = a.qss + (b * a.ssbr + rq) * a.ssrs + a.qg0 + (idx % CPR) * sper;
      qss[c][0] = *reinterpret_cast<const f32x4*>(qsp);
      qss[c][1] = *reinterpret_cast<const f32x4*>(sper >= 8 ? qsp + 4 : qsp);
      qw[c] = load8(a.qnw + h * DH + d0);
    }
  }
  bf16x8 kA[2][NC], vA[NVC], kB[2][NC], vB[NVC];
  if (kb_beg < kb_end) gload(kb_beg, kA, vA);
  __builtin_amdgcn_sched_barrier(0);

  // ---- phase 2: normalised queries -> LDS
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = tid + 256 * c, r = idx / CPR, d0 = (idx % CPR) * 8;
    bf16x8 qn = qr[c];
    if constexpr (QN) {
      const int64_t sper = a.nwidth / 16 / CPR;
      float sq = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j == 1 && sper < 8) break;
        sq += (qss[c][j][0] + qss[c][j][1]) + (qss[c][j][2] + qss[c][j][3]);
      }
      for (int64_t g = 8; g < sper; g += 4) {
        const int rq = r < Sq ? r : 0;
        const f32x4 x = *reinterpret_cast<const f32x4*>(a.qss + (b * a.ssbr + rq) * a.ssrs + a.qg0 + (idx % CPR) * sper + g);
        sq += (x[0] + x[1]) + (x[2] + x[3]);
      }
#pragma unroll
      for (int o = 1; o < CPR; o <<= 1) sq += __shfl_xor(sq, o, kWave);
      const float rq = rsqrtf(sq / (float)a.nwidth + a.neps);
      qn = norm_rope8(qr[c], rq, qw[c], f32x4{1.f, 1.f, 1.f, 1.f}, f32x4{0.f, 0.f, 0.f, 0.f}, false);
    }
    *reinterpret_cast<bf16x8*>(&Qs[r][d0]) = qn;
  }
  __syncthreads();
  bf16x8 qf[2][NC];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[qt][c] = *reinterpret_cast<const bf16x8*>(&Qs[qt * 16 + l16][c * 32 + lg * 8]);

  f32x4 oacc[2][NDT];
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int t = 0; t < NDT; ++t) oacc[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](int blk, const bf16x8 (&kf)[2][NC], const bf16x8 (&vc)[NVC]) {
#pragma unroll
    for (int p = 0; p < NVC; ++p) {
      const int cidx = lane + 64 * p, key = cidx / CPR, d0 = (cidx % CPR) * 8;
      *reinterpret_cast<bf16x8*>(&Vs[wave][key][d0]) = vc[p];
    }
    __builtin_amdgcn_wave_barrier();
    // V^T fragment of dim tile t (row = dim, k = key): lane s of a 16-lane group loads key
    // 4 lg + s / 4 (+ 16 for the upper half), dims 16 t + 4 (s % 4) .. + 3, and lane i receives
    // keys 4 lg .. 4 lg + 3 of dim 16 t + i -- the key order of the P fragment below
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    bf16x8 vfr[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const int key = lg * 4 + (l16 >> 2), dim = t * 16 + 4 * (l16 & 3);
      lds_s16x4* p0 = (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&Vs[wave][key][dim];
      lds_s16x4* p1 = (lds_s16x4*)(__attribute__((address_space(3))) bf16*)&Vs[wave][key + 16][dim];
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1);
      const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      vfr[t] = __builtin_bit_cast(bf16x8, v8);
    }
    const bool full = (blk + 1) * KB <= Sk;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float sc[2][4];
      float mloc = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) acc = mfma16(kf[kt][c], qf[qt][c], acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[e] * a.scale_log2;
          if (!full) v = (blk * KB + kt * 16 + lg * 4 + e < Sk) ? v : -INFINITY;
          sc[kt][e] = v;
          mloc = fmaxf(mloc, v);
        }
      }
      const float m_new = fmaxf(m_run[qt], group4_max(mloc));   // finite: the block has a valid key
      const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
      float psum = 0.f;
      bf16x8 pf;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pv = __builtin_amdgcn_exp2f(sc[kt][e] - m_new);
          psum += pv;
          pf[kt * 4 + e] = to_bf(pv);
        }
      l_run[qt] = l_run[qt] * alpha + group4_sum(psum);
      m_run[qt] = m_new;
#pragma unroll
      for (int t = 0; t < NDT; ++t) oacc[qt][t] = mfma16(vfr[t], pf, oacc[qt][t] * alpha);
    }
    __builtin_amdgcn_wave_barrier();  // the next block may overwrite this wave's V tile
  };

  for (int blk = kb_beg; blk < kb_end; blk += 2) {
    if (blk + 1 < kb_end) gload(blk + 1, kB, vB);
    __builtin_amdgcn_sched_barrier(0);
    process(blk, kA, vA);
    if (blk + 1 >= kb_end) break;
    if (blk + 2 < kb_end) gload(blk + 2, kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    process(blk + 1, kB, vB);
  }

  // ---- merge the four waves' states: (m, l) first, then each wave's rescaled o, summed in wave order
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
    if (lg == 0) { s_m[wave][qt * 16 + l16] = m_run[qt]; s_l[wave][qt * 16 + l16] = l_run[qt]; }
  __syncthreads();
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = qt * 16 + l16;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_m[w][q]);
    const float sc = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[qt] - mx);  // a wave without keys has m = -inf
#pragma unroll
    for (int t = 0; t < NDT; ++t)
      *reinterpret_cast<f32x4*>(&s_o[wave][q][t * 16 + lg * 4]) = oacc[qt][t] * sc;
  }
  __syncthreads();
  for (int idx = tid; idx < 32 * (DH / 4); idx += 256) {
    const int q = idx / (DH / 4), d0 = (idx % (DH / 4)) * 4;
    if (q >= Sq) continue;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_m[w][q]);
    float L = 0.f;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        L += s_l[w][q] * __builtin_amdgcn_exp2f(s_m[w][q] - mx);
        v += *reinterpret_cast<const f32x4*>(&s_o[w][q][d0]);
      }
    }
    if (a.splits > 1) {
      const int64_t row = ((int64_t)blockIdx.y * gridDim.x + bh) * a.Sq + q;
      *reinterpret_cast<f32x4*>(a.part_o + row * DH + d0) = v;
      if (d0 == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = make_float2(mx, L);
    } else {
      const float inv = L > 0.f ? 1.0f / L : 0.f;
      bf16x4 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = to_bf(v[e] * inv);
      *reinterpret_cast<bf16x4*>(a.o + b * a.o_bs + q * a.o_rs + h * a.o_hs + d0) = ov;
    }
  }
}

// ---------------------------------------------------------------------------------------
// attn_long_kernel: long query sequences (video tokens), one key segment, no mask or a key mask.
// A workgroup of 4 waves owns 128 queries of one (batch, head), 32 per wave; keys stream in
// 64-key tiles through double-buffered LDS (K and V row-major), one barrier per tile, the
// next tile's buffer loads in flight during the current tile's math.  Per wave and tile:
//   S^T [64 keys x 32 queries] = K Q^T      2 x DH/16 MFMA 32x32x16 (A = K rows from LDS,
//                                           B = the wave's queries, held in registers)
//   online softmax per query (a lane owns one query: 32 of its scores plus 32 in lane l^32)
//   O^T [DH x 32 queries] += V^T P^T        2 x 2 x DH/32 MFMA (A = V^T through transposing
//                                           LDS reads, B = P kept in registers; the key order
//                                           inside a 16-key step is permuted identically on
//                                           both operands)
// At most 256 registers per lane, so two workgroups share a CU and one's vector work fills
// the other's matrix-core gaps.  Work-groups are mapped so that all query blocks of one head
// run on the same XCD (its 4 MB L2 then holds that head's K/V once).
// KMASK: a boolean key mask shared by every query (mask query stride 0: the text padding mask
// of the cross-attention, [B, Lc] or [B, H, Lc]); each tile's 64 entries travel with the K/V
// tile as additive 0 / -inf terms in LDS (keys past Sk included).
// KW = 2 (head dim 128, a grid of at most one workgroup per CU): 8 waves in two key groups of
// 4; group g takes the tiles g, g + 2, g + 4, ... of the same 128 queries with its own LDS slots,
// so each SIMD runs two waves (one's softmax under the other's MFMAs) although the grid leaves
// one workgroup per CU, and group 1 hands its softmax state to group 0 through LDS at the end.
template <int DH, bool KMASK, int KW>
__global__ __launch_bounds__(256 * KW, 2 / KW) void attn_long_kernel(AttnArgs a, int nqb) {
  constexpr int NTH = 256 * KW;          // threads; 32 queries per wave, KW waves per query group
  constexpr int BN = 64;                 // keys per tile
  constexpr int KS = DH / 16;            // 16-wide k-steps of S^T = K Q^T
  constexpr int DT = DH / 32;            // 32-row dim tiles of O^T
  constexpr int CPR = DH / 8;            // 16-byte chunks per K/V row
  constexpr int NCH = BN * CPR / NTH;    // chunks of K (and of V) per thread per tile
  // Head dim 128: K and V tiles arrive by direct-to-LDS buffer loads (no register staging, no
  // LDS stores by the waves) into unpadded 256-byte rows whose 16-byte chunks are XOR-swizzled:
  // chunk c of K row r at c ^ (r & 15) (the 16-byte fragment reads of 16 rows then hit 16
  // distinct bank groups), of V row r at c ^ 4 (r & 3) (the transposing reads of 4 rows x 4
  // chunks then cover the 64 banks once).  Head dim 64: the tiles go through registers into
  // padded rows -- K 144 bytes, V 192 mod 256, so the transposing reads of 8 rows x 64 bytes
  // fill the banks twice exactly.
  constexpr bool DMA = DH == 128;
  static_assert(KW == 1 || (KW == 2 && DMA), "key groups need the direct-to-LDS path");
  constexpr int KLD = DH + 8, VLD = DH == 128 ? 160 : 96;
  __shared__ bf16 Ks[2][DMA ? 1 : BN][DMA ? 8 : KLD];
  __shared__ bf16 Vs[2][DMA ? 1 : BN][DMA ? 8 : VLD];
  __shared__ __attribute__((aligned(1024))) bf16 Kd[DMA ? 2 : 1][KW][DMA ? BN * DH : 8];
  __shared__ __attribute__((aligned(1024))) bf16 Vd[DMA ? 2 : 1][KW][DMA ? BN * DH : 8];
  __shared__ __attribute__((aligned(16))) float Mb[KMASK ? 2 : 1][KW][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3;   // wave: query group
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int kg = KW == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 8);   // key group
  const int gtid = KW == 1 ? tid : tid & 255;                               // thread within it
  const int l32 = lane & 31, hh = lane >> 5;
  // XCD-aware task order: workgroup i runs on XCD i % 8; give each XCD a contiguous range of
  // (head, query block) tasks so that a head's query blocks share that XCD's L2
  const int nwg = gridDim.x;
  int task = blockIdx.x;
  if ((nwg & 7) == 0) task = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int bh = task / nqb, qb = task - bh * nqb;
  const uint32_t H32 = (uint32_t)a.H;
  const uint32_t b = (uint32_t)bh / H32, h = (uint32_t)bh - b * H32;
  const int Sq = (int)a.Sq, Sk = (int)a.Sk;
  const bf16* qbase = a.q + b * a.q_bs + h * a.q_hs;
  const bf16* kbase = a.k0 + b * a.k0_bs + h * a.k0_hs;
  const bf16* vbase = a.v0 + b * a.v0_bs + h * a.v0_hs;

  // the wave's 32 queries as B operands: lane -> query l32, dims 16s + 8hh .. +7
  const int q = qb * 128 + wave * 32 + l32;
  const int qc = q < Sq ? q : 0;
  bf16x8 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = load8(qbase + (int64_t)qc * a.q_rs + ks * 16 + hh * 8);

  // K/V tiles come in through raw buffer loads: the descriptor (scalar registers) is rebuilt
  // per tile over the rows from the tile's first key to Sk, so rows past the end (and whole
  // tiles past the end) read as zero and each thread keeps only 32-bit row offsets.  Every row
  // offset goes into the per-lane (vector) offset: the range check covers the vector and
  // instruction offsets only, not the scalar one, so a row placed there would be read past Sk.
  const uint32_t krs = (uint32_t)a.k0_rs * 2u, vrs = (uint32_t)a.v0_rs * 2u;   // bytes per row
  // direct loads: instruction n of wave w writes rows 4 (w + 4n) .. + 3 of the slot (1 KB;
  // lane j -> row + j / 16, chunk slot j % 16) and lane j fetches the chunk that belongs there
  const int dr = lane >> 4;
  const uint32_t dk = (uint32_t)dr * krs + (uint32_t)(((lane & 15) ^ ((4 * wave + dr) & 15)) * 16);
  const uint32_t dv = (uint32_t)dr * vrs + (uint32_t)(((lane & 15) ^ (4 * dr)) * 16);
  auto dma_kv = [&](int t, int buf) {
    if constexpr (DMA) {
      const int k0 = t * BN, left = Sk - k0 > 0 ? Sk - k0 : 0;
      const auto rk = buffer_rsrc(kbase + (int64_t)k0 * a.k0_rs, (uint32_t)left * krs);
      const auto rv = buffer_rsrc(vbase + (int64_t)k0 * a.v0_rs, (uint32_t)left * vrs);
#pragma unroll
      for (int n = 0; n < BN / 16; ++n) {
        const int r0 = 4 * (wv + 4 * n);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)&Kd[buf][kg][r0 * DH], 16,
                                                 dk + (uint32_t)r0 * krs, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)&Vd[buf][kg][r0 * DH], 16,
                                                 dv + (uint32_t)r0 * vrs, 0, 0, 0);
      }
    }
  };
  // register path: chunk j of a thread is key tid / CPR + j * (NTH / CPR), dims (tid % CPR) * 8
  // .. + 7: one per-lane offset plus the j step
  const uint32_t koff = (uint32_t)(tid / CPR) * krs + (uint32_t)(tid % CPR) * 16u;
  const uint32_t voff = (uint32_t)(tid / CPR) * vrs + (uint32_t)(tid % CPR) * 16u;
  bf16x8 kr[DMA ? 1 : NCH], vr[DMA ? 1 : NCH];
  auto gload_kv = [&](int t) {
    if constexpr (!DMA) {
      const int k0 = t * BN, left = Sk - k0 > 0 ? Sk - k0 : 0;
      const auto rk = buffer_rsrc(kbase + (int64_t)k0 * a.k0_rs, (uint32_t)left * krs);
      const auto rv = buffer_rsrc(vbase + (int64_t)k0 * a.v0_rs, (uint32_t)left * vrs);
#pragma unroll
      for (int j = 0; j < NCH; ++j) kr[j] = buffer_load8(rk, koff + (uint32_t)j * (NTH / CPR) * krs);
#pragma unroll
      for (int j = 0; j < NCH; ++j) vr[j] = buffer_load8(rv, voff + (uint32_t)j * (NTH / CPR) * vrs);
    }
  };
  auto lstore_kv = [&](int buf) {
    if constexpr (!DMA) {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = tid + NTH * j, key = c / CPR, d0 = (c % CPR) * 8;
        *reinterpret_cast<bf16x8*>(&Ks[buf][key][d0]) = kr[j];
        *reinterpret_cast<bf16x8*>(&Vs[buf][key][d0]) = vr[j];
      }
    }
  };
  // key mask of tile t (thread tid < BN: key t * BN + tid), as an additive term
  const uint8_t* mrow = KMASK ? reinterpret_cast<const uint8_t*>(a.mask) + b * a.mbs + h * a.mhs : nullptr;
  // (the raw byte is kept until the LDS store, so that the load's wait lands there)
  int mr = 0;
  auto gload_m = [&](int t) {
    if constexpr (KMASK) {
      const int key = t * BN + (gtid & (BN - 1));
      mr = key < Sk ? (int)mrow[key] : 0;
    }
  };
  auto lstore_m = [&](int buf) {
    if constexpr (KMASK) {
      if (gtid < BN) Mb[buf][kg][gtid] = mr ? 0.f : -INFINITY;
    }
  };
  // A operand of the PV product (V^T: row = dim, k = key) straight from the row-major tile
  // with two transposing LDS reads (ds_read_b64_tr_b16).  Within each 16-lane group, lane i
  // receives element i % 4 of the 8-byte loads of lanes i / 4 + 4e (e = 0..3); so lane s of a
  // group loads key k0 + s / 4, dims dbase + 4 (s % 4) .. + 3, and lane i ends up with keys
  // k0 .. k0 + 3 of dim dbase + i.  Lanes 0-15 / 16-31 take dims 0-15 / 16-31 of the 32-dim
  // tile, lanes 32-63 the same dims for keys 4 further (their k-half of the MFMA).
  // The lane-dependent parts of both fragments' LDS addresses are computed once (per k-step /
  // dim tile where the swizzle makes them differ); with the tile's buffer a compile-time
  // constant every read is a lane register plus an immediate offset.
  typedef __attribute__((address_space(3))) bf16 lds_bf16;
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int s16 = lane & 15;
  const int koff_l = l32 * KLD + hh * 8;
  const int voff_l = (4 * hh + (s16 >> 2)) * VLD + 16 * ((lane >> 4) & 1) + 4 * (s16 & 3);
  int kofs[DMA ? KS : 1], vofs[DMA ? DT : 1];
  if constexpr (DMA) {
    // K: row l32 (+ 32 kt), chunk 2 ks + hh at (2 ks + hh) ^ (l32 & 15)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kofs[ks] = l32 * DH + (((2 * ks + hh) ^ (l32 & 15)) * 8);
    // V: row 4 hh + s/4 (+ k0), dims 32 d + 16 ((lane >> 4) & 1) + 4 (s & 3): chunk 4 d + e with
    // e = 2 ((lane >> 4) & 1) + (s & 3) / 2 at 4 (d ^ (s / 4)) + e (the row's r & 3 is s / 4),
    // 8 bytes into it for odd s
    const int e = 2 * ((lane >> 4) & 1) + ((s16 & 3) >> 1);
#pragma unroll
    for (int d = 0; d < DT; ++d)
      vofs[d] = (4 * hh + (s16 >> 2)) * DH + (4 * (d ^ (s16 >> 2)) + e) * 8 + (s16 & 1) * 4;
  }
  auto vfrag = [&](int buf, int k0, int d) {
    const lds_bf16* p0;
    if constexpr (DMA) p0 = (const lds_bf16*)&Vd[buf][kg][0] + vofs[d] + k0 * DH;
    else p0 = (const lds_bf16*)&Vs[buf][0][0] + voff_l + k0 * VLD + d * 32;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0 + 8 * (DMA ? DH : VLD)));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  };
  // S^T of a tile: register r of half kt holds key kt*32 + 8*(r/4) + 4*hh + r%4 of the lane's
  // query; the two halves are independent MFMA chains, interleaved
  auto kfrag = [&](int buf, int kt, int ks) {
    const lds_bf16* p;
    if constexpr (DMA) p = (const lds_bf16*)&Kd[buf][kg][0] + kofs[ks] + kt * 32 * DH;
    else p = (const lds_bf16*)&Ks[buf][0][0] + koff_l + kt * 32 * KLD + ks * 16;
    return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(p);
  };
  f32x16 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) acc[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = a.scale_log2;
  const int ntiles_kw = (Sk + BN - 1) / BN;
  const int nfull_kw = KMASK ? ntiles_kw : Sk / BN;

  // one 64-key tile t of this key group from LDS buffer BUF; TAIL (the partial last tile
  // without a key mask) sets the scores of keys past Sk to -inf, so full tiles carry no
  // per-score masking.  The group's next tile (t + KW) goes to the other buffer first, which the
  // last barrier released (zeros past Sk).
  auto compute = [&](int t, auto tail_tag, auto buf_tag) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    constexpr int buf = decltype(buf_tag)::value;
    f32x16 st[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) st[kt] = mfma32(kfrag(buf, kt, ks), qf[ks], st[kt]);
    if constexpr (KMASK) {
      // registers 4g..4g+3 of half kt: keys kt*32 + 8g + 4hh .. + 3
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const f32x4 m4 = *reinterpret_cast<const f32x4*>(&Mb[buf][kg][kt * 32 + 8 * g4 + 4 * hh]);
#pragma unroll
          for (int e = 0; e < 4; ++e) st[kt][4 * g4 + e] += m4[e];
        }
    } else if constexpr (TAIL) {
      const int kleft = Sk - t * BN - 4 * hh;   // keys of this tile below Sk, relative to the lane's first
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          st[kt][r] = kt * 32 + 8 * (r / 4) + (r % 4) < kleft ? st[kt][r] : -INFINITY;
    }
    // online softmax (log2 domain).  The running max only moves when a score exceeds it by
    // more than 2^8 (or on the first tile), so the accumulator rescale is skipped on most
    // tiles; p <= 2^8 in between is exact in fp32 and bf16 keeps its relative precision.
    float mraw = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mraw = fmaxf(mraw, st[kt][r]);
    mraw = max_xor32(mraw);
    const float mloc = mraw * sl2;   // sl2 > 0
    if (__any(mloc > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // max unchanged: 1; -inf: 0
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DT; ++d) acc[d] *= alpha;
      m_run = m_new;
    }
    // (a query whose keys so far are all masked keeps m_run = -inf: its p are exp2(-inf) = 0)
    const float m_use = KMASK && m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
    bf16x8 pf[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kt][r], sl2, -m_use));
        psum += pv;
        pf[kt][r / 8][r % 8] = to_bf(pv);
      }
    psum = sum_xor32(psum);
    l_run += psum;
    // O^T += V^T P^T: k-step c of half kt covers keys kt*32 + 16c + {4hh..4hh+3, 8+4hh..8+4hh+3}
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int d = 0; d < DT; ++d) acc[d] = mfma32(vfrag(buf, kt * 32 + 16 * c, d), pf[kt][c], acc[d]);
  };
  auto prefetch = [&](int t, int buf) {
    dma_kv(t, buf);
    gload_kv(t);
    gload_m(t);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto finish = [&](int buf) {
    lstore_kv(buf);
    lstore_m(buf);
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0): the next tile landed
    __syncthreads();
  };
  auto tile = [&](int t, auto tail_tag, auto buf_tag) {
    constexpr int buf = decltype(buf_tag)::value;
    prefetch(t + 1, buf ^ 1);
    compute(t, tail_tag, buf_tag);
    finish(buf ^ 1);
  };
  // KW = 2: stage s holds tile 2 s + kg of each key group; a group whose tile is past the end
  // (odd tile count) only loads zeros and meets the barriers
  auto stage = [&](int s, auto buf_tag) {
    constexpr int buf = decltype(buf_tag)::value;
    const int tg = KW * s + kg;
    prefetch(tg + KW, buf ^ 1);
    if (tg < nfull_kw) compute(tg, std::false_type{}, buf_tag);
    else if (tg < ntiles_kw) compute(tg, std::true_type{}, buf_tag);
    finish(buf ^ 1);
  };

  const int ntiles = ntiles_kw;
  const int nfull = nfull_kw;   // tiles whose keys are all below Sk (or masked)
  prefetch(kg, 0);
  finish(0);
  using F = std::false_type;
  using T = std::true_type;
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  if constexpr (KW == 1) {
    int t = 0;
    for (; t + 1 < nfull; t += 2) {
      tile(t, F{}, B0{});
      tile(t + 1, F{}, B1{});
    }
    if (t < nfull) {
      tile(t, F{}, B0{});
      if (t + 1 < ntiles) tile(t + 1, T{}, B1{});
    } else if (t < ntiles) {
      tile(t, T{}, B0{});
    }
  } else {
    const int nst = (ntiles + KW - 1) / KW;
    int s = 0;
    for (; s + 1 < nst; s += 2) {
      stage(s, B0{});
      stage(s + 1, B1{});
    }
    if (s < nst) stage(s, B0{});
    // group 1 parks its (m, l, O^T) in the K/V slots (free after the last barrier: the loads of
    // tiles past the end have landed), group 0 merges them into its own
    float* park = reinterpret_cast<float*>(&Kd[0][0][0]);   // DT * 16 floats per lane, per wave
    float* pml = reinterpret_cast<float*>(&Vd[0][0][0]);    // (m, l) per lane, per wave
    if (kg == 1) {
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) park[((wave * DT + d) * 16 + r) * 64 + lane] = acc[d][r];
      pml[(wave * 2) * 64 + lane] = m_run;
      pml[(wave * 2 + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (kg == 1) return;   // no barrier follows
    const float m1 = pml[(wave * 2) * 64 + lane], l1 = pml[(wave * 2 + 1) * 64 + lane];
    const float mm = fmaxf(m_run, m1);
    const float a0 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mm);
    const float a1 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[d][r] = acc[d][r] * a0 + park[((wave * DT + d) * 16 + r) * 64 + lane] * a1;
    l_run = l_run * a0 + l1 * a1;
  }

  if (q >= Sq) return;
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  bf16* op = a.o + b * a.o_bs + (int64_t)q * a.o_rs + h * a.o_hs;
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {   // registers 4g..4g+3: dims d*32 + 8g + 4hh .. +3
      bf16x4 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = to_bf(acc[d][4 * g + e] * inv);
      *reinterpret_cast<bf16x4*>(op + d * 32 + 8 * g + 4 * hh) = ov;
    }
}

// Merge of the key-split partials: one thread per (b*h, q, 4 channels), splits in order.
// Index math in 32 bits (the host checks that the thread count fits) with the head dim a
// template constant where it is 64 or 128 (DHC = 0: at run time): 64-bit divisions cost
// dozens of instructions each on the kernel's one wave per CU.  Up to MAXS splits are loaded
// before the first use (one memory round trip); more splits (MAXS = 0) take the looped form.
template <int MAXS, int DHC>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a, int dh_rt, uint32_t total) {
  const uint32_t idx = blockIdx.x * 64u + threadIdx.x;
  if (idx >= total) return;
  const uint32_t DH = DHC ? (uint32_t)DHC : (uint32_t)dh_rt, nd4 = DH / 4;
  const uint32_t d0 = (idx % nd4) * 4u, rq = idx / nd4;   // rq = bh * Sq + q
  const uint32_t Sq = (uint32_t)a.Sq, H = (uint32_t)a.H;
  const uint32_t q = rq % Sq, bh = rq / Sq, b = bh / H, h = bh - b * H;
  const uint32_t plane = total / nd4;                      // BH * Sq rows per split
  const int S = a.splits;
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  if constexpr (MAXS > 0) {
    float2 ml[MAXS];
    f32x4 po[MAXS];
#pragma unroll
    for (int z = 0; z < MAXS; ++z) {
      const int64_t row = (int64_t)(z < S ? z : S - 1) * plane + rq;
      ml[z] = *reinterpret_cast<const float2*>(a.part_ml + row * 2);
      po[z] = *reinterpret_cast<const f32x4*>(a.part_o + row * DH + d0);
    }
    __builtin_amdgcn_sched_barrier(0);
    float mx = -INFINITY;
#pragma unroll
    for (int z = 0; z < MAXS; ++z)
      if (z < S) mx = fmaxf(mx, ml[z].x);
    if (mx != -INFINITY) {
#pragma unroll
      for (int z = 0; z < MAXS; ++z)
        if (z < S) {
          const float w = __builtin_amdgcn_exp2f(ml[z].x - mx);   // an empty split has m = -inf -> 0
          L += ml[z].y * w;
          o += po[z] * w;
        }
    }
  } else {
    float mx = -INFINITY;
    for (int z = 0; z < S; ++z) mx = fmaxf(mx, a.part_ml[((int64_t)z * plane + rq) * 2]);
    if (mx != -INFINITY) {
      for (int z = 0; z < S; ++z) {
        const int64_t row = (int64_t)z * plane + rq;
        const float w = __builtin_amdgcn_exp2f(a.part_ml[row * 2] - mx);
        L += a.part_ml[row * 2 + 1] * w;
        o += *reinterpret_cast<const f32x4*>(a.part_o + row * DH + d0) * w;
      }
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  bf16x4 ov;
#pragma unroll
  for (int e = 0; e < 4; ++e) ov[e] = to_bf(o[e] * inv);
  *reinterpret_cast<bf16x4*>(a.o + b * a.o_bs + q * a.o_rs + h * a.o_hs + d0) = ov;
}

template <int MAXS>
static void launch_combine_s(const AttnArgs& a, int dh, uint32_t total, hipStream_t s) {
  const dim3 grid((total + 63) / 64);
  if (dh == 64) FAM_LAUNCH((attn_combine_kernel<MAXS, 64>), grid, dim3(64), 0, s, a, dh, total);
  else if (dh == 128) FAM_LAUNCH((attn_combine_kernel<MAXS, 128>), grid, dim3(64), 0, s, a, dh, total);
  else FAM_LAUNCH((attn_combine_kernel<MAXS, 0>), grid, dim3(64), 0, s, a, dh, total);
}

// ---------------------------------------------------------------------------------------
template <int DH>
__global__ __launch_bounds__(256) void attn_tiled_kernel(AttnArgs a) {
  constexpr int NW = 4;
  constexpr int NC = (DH + 31) / 32;
  constexpr int NDT = (DH + 15) / 16;
  constexpr int DP = NC * 32 + 8;
  constexpr int VROWS = NDT * 16;
  __shared__ bf16 Ks[KB][DP];
  __shared__ bf16 Vt[VROWS][KB + 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t bh = blockIdx.y, b = bh / a.H, h = bh - b * a.H;
  const int64_t qi = (int64_t)blockIdx.x * 16 * NW + wave * 16 + l16;
  const bool qvalid = qi < a.Sq;

  bf16x8 qf[NC];
  const bf16* qbase = a.q + b * a.q_bs + h * a.q_hs;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d0 = c * 32 + lg * 8;
    qf[c] = load8_if(qvalid && d0 < DH, qbase + qi * a.q_rs + d0, qbase);
  }
  const SegRows krows = key_rows(a, b, h), vrows = val_rows(a, b, h);
  const bf16* ksafe = krows.row(0);
  const bf16* vsafe = vrows.row(0);
  f32x4 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int64_t kb = 0; kb < a.Sk; kb += KB) {
    for (int c = tid; c < KB * (DH / 8); c += NW * 64) {
      const int key = c / (DH / 8), d0 = (c % (DH / 8)) * 8;
      const int64_t kk = kb + key;
      const bool ok = kk < a.Sk;
      const bf16x8 kv = load8_if(ok, krows.row(ok ? kk : 0) + d0, ksafe);
      const bf16x8 vv = load8_if(ok, vrows.row(ok ? kk : 0) + d0, vsafe);
      *reinterpret_cast<bf16x8*>(&Ks[key][d0]) = kv;
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[d0 + e][key] = vv[e];
    }
    __syncthreads();
    float s[2][4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d0 = c * 32 + lg * 8;
        const bf16x8 kfr = (d0 < DH) ? *reinterpret_cast<const bf16x8*>(&Ks[kt * 16 + l16][d0]) : zero8();
        sacc = mfma16(kfr, qf[c], sacc);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) s[kt][e] = score(a, sacc[e], b, h, qi, qvalid, kb + kt * 16 + lg * 4 + e);
    }
    const bf16x8 pf = softmax_update<NDT>(s, m_run, l_run, oacc);
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

static int64_t rup(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Waves per workgroup: enough to split long key runs, few enough that the per-wave state
// (query fragments, accumulators, the next block's K/V) fits the register file without spills.
template <int DH, int QT, bool QN, bool KN>
static void launch_short_qk(const AttnArgs& a, int64_t nkb, dim3 grid, hipStream_t s) {
  constexpr bool wide = DH >= 128 && QT >= 2;
  if (nkb <= 1) FAM_LAUNCH((attn_short_kernel<DH, QT, 1, QN, KN>), grid, dim3(64), 0, s, a);
  else if (nkb <= 2) FAM_LAUNCH((attn_short_kernel<DH, QT, 2, QN, KN>), grid, dim3(128), 0, s, a);
  else if (nkb <= 4 || wide) FAM_LAUNCH((attn_short_kernel<DH, QT, 4, QN, KN>), grid, dim3(256), 0, s, a);
  else FAM_LAUNCH((attn_short_kernel<DH, QT, (wide ? 4 : 8), QN, KN>), grid, dim3((wide ? 4 : 8) * 64), 0, s, a);
}

template <int DH, int QT>
static void launch_short_q(const AttnArgs& a, int64_t nkb, dim3 grid, hipStream_t s) {
  if constexpr (DH >= 64 && QT <= 2) {
    if (a.qss != nullptr || a.kss != nullptr) {
      if (a.kss == nullptr) launch_short_qk<DH, QT, true, false>(a, nkb, grid, s);
      else if (a.qss == nullptr) launch_short_qk<DH, QT, false, true>(a, nkb, grid, s);
      else launch_short_qk<DH, QT, true, true>(a, nkb, grid, s);
      return;
    }
  }
  constexpr bool wide = DH >= 128 && QT >= 2;
  if (nkb <= 1) FAM_LAUNCH((attn_short_kernel<DH, QT, 1>), grid, dim3(64), 0, s, a);
  else if (nkb <= 2) FAM_LAUNCH((attn_short_kernel<DH, QT, 2>), grid, dim3(128), 0, s, a);
  else if (nkb <= 4 || wide) FAM_LAUNCH((attn_short_kernel<DH, QT, 4>), grid, dim3(256), 0, s, a);
  else FAM_LAUNCH((attn_short_kernel<DH, QT, (wide ? 4 : 8)>), grid, dim3((wide ? 4 : 8) * 64), 0, s, a);
}

template <int DH, int NW, int NV, int NSS>
static void launch_small_mk(const AttnArgs& a, dim3 grid, hipStream_t s) {
  if (a.mask_kind == FAM_MASK_NONE) FAM_LAUNCH((attn_small_kernel<DH, NW, NV, NSS, 0>), grid, dim3(NW * 64), 0, s, a);
  else if (a.mask_kind == FAM_MASK_BOOL) FAM_LAUNCH((attn_small_kernel<DH, NW, NV, NSS, 1>), grid, dim3(NW * 64), 0, s, a);
  else FAM_LAUNCH((attn_small_kernel<DH, NW, NV, NSS, 2>), grid, dim3(NW * 64), 0, s, a);
}
template <int DH, int NW, int NV>
static void launch_small_nv(const AttnArgs& a, bool qn, dim3 grid, hipStream_t s) {
  if (qn) launch_small_mk<DH, NW, NV, 8>(a, grid, s);
  else launch_small_mk<DH, NW, NV, 0>(a, grid, s);
}
template <int DH, int NW>
static void launch_small_nw(const AttnArgs& a, bool qn, int64_t bh, int nqc, hipStream_t s) {
  // a (head, query chunk) over 8, 4 or 2 CUs (output-dim eighths / quarters / halves) while that
  // keeps the grid within one round: each slice's workgroup repeats the scores but runs 1/NV of
  // P V and of the merge (eighths only at DH = 128: a slice keeps at least one 16-dim MFMA tile;
  // halves for the video prefill's 24 heads x 4 query chunks)
  const int64_t units = bh * nqc;
  if constexpr (DH == 128) {
    if (units <= 32) {
      launch_small_nv<DH, NW, 8>(a, qn, dim3((unsigned)bh, 8, (unsigned)nqc), s);
      return;
    }
  }
  if (units <= 64) launch_small_nv<DH, NW, 4>(a, qn, dim3((unsigned)bh, 4, (unsigned)nqc), s);
  else if (units <= 128) launch_small_nv<DH, NW, 2>(a, qn, dim3((unsigned)bh, 2, (unsigned)nqc), s);
  else launch_small_nv<DH, NW, 1>(a, qn, dim3((unsigned)bh, 1, (unsigned)nqc), s);
}
template <int DH>
static void launch_small(const AttnArgs& a, int nw, bool qn, int64_t bh, hipStream_t s) {
  const int nqc = (int)((a.Sq + 31) / 32);   // query chunks (one unless more than 32 queries)
  if (nw <= 2) launch_small_nw<DH, 2>(a, qn, bh, nqc, s);
  else if (nw <= 4) launch_small_nw<DH, 4>(a, qn, bh, nqc, s);
  else if (nw <= 6) launch_small_nw<DH, 6>(a, qn, bh, nqc, s);
  else launch_small_nw<DH, 8>(a, qn, bh, nqc, s);
}

template <int DH>
static void launch_dh(const AttnArgs& a, int64_t bh, hipStream_t s) {
  if constexpr (DH == 64 || DH == 128) {
    // the action tokens over their own keys: one workgroup per head, LDS-staged q/k/v
    if (a.Sq <= 32 && a.Sk >= 1 && a.Sk <= 32 && a.sk0 == a.Sk && a.mask_kind == FAM_MASK_NONE && a.splits == 1 &&
        (a.qss == nullptr) == (a.kss == nullptr)) {
      if (a.qss) FAM_LAUNCH((attn_self_kernel<DH, true>), dim3((unsigned)bh), dim3(256), 0, s, a);
      else FAM_LAUNCH((attn_self_kernel<DH, false>), dim3((unsigned)bh), dim3(256), 0, s, a);
      return;
    }
  }
  if constexpr (DH == 64 || DH == 128) {
    // up to 32 queries over up to 256 keys in one workgroup per head (no key splits): the MoT
    // joint attention over [video K/V ; action K/V], a short context; up to 128 queries without
    // on-load normalisation as chunks of 32 (grid.z; the video prefill's 98 tokens over 98 / 129
    // keys) (its mask entries are buffer loads with 32-bit offsets over one (batch, head) span)
    const int64_t msz = a.mask_kind == FAM_MASK_BOOL ? 1 : (a.mask_kind == FAM_MASK_ADD_F32 ? 4 : 2);
    const bool mask_fits = a.mask_kind == FAM_MASK_NONE ||
                           (a.mqs >= 0 && ((a.Sq - 1) * a.mqs + a.Sk) * msz < ((int64_t)1 << 31));
    if ((a.Sq <= 32 || (a.Sq <= 128 && a.qss == nullptr)) && a.Sk >= 1 && a.Sk <= 256 && a.splits == 1 &&
        a.kss == nullptr && mask_fits && (a.qss == nullptr || a.nwidth <= 4096)) {
      const int nw = (int)((a.Sk + KB - 1) / KB);
      launch_small<DH>(a, nw, a.qss != nullptr, bh, s);
      return;
    }
    // up to 32 queries over one long unmasked key segment (the context)
    if (a.Sq <= 32 && a.sk0 == a.Sk && a.mask_kind == FAM_MASK_NONE && a.kss == nullptr) {
      const dim3 grid((unsigned)bh, (unsigned)a.splits);
      if (a.qss) FAM_LAUNCH((attn_cross_kernel<DH, true>), grid, dim3(256), 0, s, a);
      else FAM_LAUNCH((attn_cross_kernel<DH, false>), grid, dim3(256), 0, s, a);
      return;
    }
  }
  // (Dh = 128 with more than 32 queries would not fit the short kernel's registers)
  if (a.Sq <= 32 || (a.Sq <= 64 && DH < 128)) {
    const int64_t nkb = ((a.Sk + KB - 1) / KB + a.splits - 1) / a.splits;  // key blocks per workgroup
    const dim3 grid((unsigned)bh, (unsigned)a.splits);
    if (a.Sq <= 16) launch_short_q<DH, 1>(a, nkb, grid, s);
    else if (a.Sq <= 32) launch_short_q<DH, 2>(a, nkb, grid, s);
    else launch_short_q<DH, 4>(a, nkb, grid, s);
  } else {
    if constexpr (DH == 64 || DH == 128) {
      // (buffer loads address a head's K and V rows with 32-bit byte offsets)
      const bool fits32 = a.Sk * a.k0_rs * 2 < ((int64_t)1 << 31) && a.Sk * a.v0_rs * 2 < ((int64_t)1 << 31);
      const bool kmask = a.mask_kind == FAM_MASK_BOOL && a.mqs == 0;
      if (a.sk0 == a.Sk && (a.mask_kind == FAM_MASK_NONE || kmask) && a.Sk >= 1 && fits32 && a.k0_rs >= DH &&
          a.v0_rs >= DH) {
        const int nqb = (int)((a.Sq + 127) / 128);
        const dim3 grid((unsigned)(nqb * bh));
        // a grid of at most one workgroup per CU runs each workgroup as two key groups of 4 waves
        // (two waves per SIMD); more workgroups share the CUs two by two instead
        if constexpr (DH == 128) {
          if (nqb * bh <= fam_host::device_cus()) {
            if (kmask) FAM_LAUNCH((attn_long_kernel<DH, true, 2>), grid, dim3(512), 0, s, a, nqb);
            else FAM_LAUNCH((attn_long_kernel<DH, false, 2>), grid, dim3(512), 0, s, a, nqb);
            return;
          }
        }
        if (kmask) FAM_LAUNCH((attn_long_kernel<DH, true, 1>), grid, dim3(256), 0, s, a, nqb);
        else FAM_LAUNCH((attn_long_kernel<DH, false, 1>), grid, dim3(256), 0, s, a, nqb);
        return;
      }
    }
    const dim3 grid((unsigned)(rup(a.Sq, 64) / 64), (unsigned)bh);
    FAM_LAUNCH((attn_tiled_kernel<DH>), grid, dim3(256), 0, s, a);
  }
}

}  // namespace fam

using namespace fam;

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
  const int64_t bh = d->batch * d->heads;
  FAM_REQUIRE(bh <= 65535 || d->sq <= 64, FAM_ERR_UNSUPPORTED, "fam_attention: batch*heads must be <= 65535");
  FAM_REQUIRE(d->num_splits >= 0 && d->num_splits <= 64, FAM_ERR_INVALID_ARG, "fam_attention: num_splits in [0, 64]");
  const bool short_q = d->sq <= 32 || (d->sq <= 64 && Dh < 128);
  FAM_REQUIRE(d->num_splits <= 1 || (short_q && d->part_o && d->part_ml && fam_host::aligned16(d->part_o) &&
                                     (reinterpret_cast<uintptr_t>(d->part_ml) & 7u) == 0),
              FAM_ERR_INVALID_ARG, "fam_attention: key splits need Sq <= 32 (<= 64 for Dh < 128) and 16-byte aligned partial buffers");
  if (d->qk_norm) {
    FAM_REQUIRE(short_q && (Dh == 64 || Dh == 128) && d->sq <= 32, FAM_ERR_UNSUPPORTED,
                "fam_attention: q/k normalisation needs the short-query path (Sq <= 32) and head_dim 64 or 128");
    FAM_REQUIRE(d->q_sumsq || d->k_sumsq, FAM_ERR_INVALID_ARG, "fam_attention: qk_norm without sums of squares");
    FAM_REQUIRE(d->norm_width >= 1024 && d->norm_width % 1024 == 0 && d->ss_row_stride % 4 == 0 &&
                    d->q_group0 % 4 == 0 && d->k_group0 % 4 == 0 && d->ss_row_stride >= d->norm_width / 16 &&
                    d->ss_batch_rows >= 0,
                FAM_ERR_INVALID_ARG, "fam_attention: norm_width must be a multiple of 1024, strides/groups multiples of 4");
    FAM_REQUIRE(d->heads * Dh <= d->norm_width, FAM_ERR_INVALID_ARG, "fam_attention: heads*head_dim exceeds norm_width");
    FAM_REQUIRE(d->q_group0 >= 0 && d->k_group0 >= 0 && d->q_group0 + d->norm_width / 16 <= d->ss_row_stride &&
                    d->k_group0 + d->norm_width / 16 <= d->ss_row_stride,
                FAM_ERR_INVALID_ARG, "fam_attention: the q/k column groups must lie inside a sums-of-squares row");
    FAM_REQUIRE((!d->q_sumsq || (d->q_norm_w && fam_host::aligned16(d->q_norm_w) && fam_host::aligned16(d->q_sumsq))) &&
                    (!d->k_sumsq || (d->k_norm_w && fam_host::aligned16(d->k_norm_w) && fam_host::aligned16(d->k_sumsq))),
                FAM_ERR_INVALID_ARG, "fam_attention: normalised side needs its 16-byte aligned weight and sums");
    FAM_REQUIRE(!d->k_sumsq || d->sk1 == 0, FAM_ERR_UNSUPPORTED, "fam_attention: k normalisation needs one key segment");
    FAM_REQUIRE((d->rope_cos == nullptr) == (d->rope_sin == nullptr), FAM_ERR_INVALID_ARG,
                "fam_attention: rope_cos and rope_sin must both be given or both be null");
    FAM_REQUIRE(!d->rope_cos || (fam_host::aligned16(d->rope_cos) && fam_host::aligned16(d->rope_sin) &&
                                 d->rope_row_stride % 4 == 0 && d->rope_row_stride >= Dh / 2),
                FAM_ERR_INVALID_ARG, "fam_attention: RoPE tables need 16-byte alignment and a row stride multiple of 4");
  }
  if (d->batch == 0 || d->sq == 0) return FAM_OK;

  AttnArgs a{};
  a.q = (const bf16*)d->q; a.q_bs = d->q_bs; a.q_rs = d->q_rs; a.q_hs = d->q_hs;
  a.k0 = (const bf16*)d->k0; a.k0_bs = d->k0_bs; a.k0_rs = d->k0_rs; a.k0_hs = d->k0_hs;
  a.v0 = (const bf16*)d->v0; a.v0_bs = d->v0_bs; a.v0_rs = d->v0_rs; a.v0_hs = d->v0_hs;
  a.k1 = (const bf16*)d->k1; a.k1_bs = d->k1_bs; a.k1_rs = d->k1_rs; a.k1_hs = d->k1_hs;
  a.v1 = (const bf16*)d->v1; a.v1_bs = d->v1_bs; a.v1_rs = d->v1_rs; a.v1_hs = d->v1_hs;
  a.o = (bf16*)d->o; a.o_bs = d->o_bs; a.o_rs = d->o_rs; a.o_hs = d->o_hs;
  a.H = d->heads; a.Sq = d->sq; a.sk0 = d->sk0; a.Sk = d->sk0 + d->sk1;
  a.scale_log2 = d->scale * kLog2e;
  a.mask = d->mask; a.mask_kind = d->mask_kind; a.mbs = d->mask_bs; a.mhs = d->mask_hs; a.mqs = d->mask_qs;
  a.splits = d->num_splits > 1 ? d->num_splits : 1;
  a.part_o = d->part_o; a.part_ml = d->part_ml;
  if (d->qk_norm) {
    a.qss = d->q_sumsq; a.kss = d->k_sumsq; a.ssrs = d->ss_row_stride; a.ssbr = d->ss_batch_rows;
    a.qg0 = d->q_group0; a.kg0 = d->k_group0; a.nwidth = d->norm_width;
    a.qnw = (const bf16*)d->q_norm_w; a.knw = (const bf16*)d->k_norm_w; a.neps = d->norm_eps;
    a.rcs = d->rope_cos; a.rsn = d->rope_sin; a.rrs = d->rope_row_stride;
  }
  hipStream_t s = (hipStream_t)stream;
  switch (Dh) {
    case 8: launch_dh<8>(a, bh, s); break;
    case 16: launch_dh<16>(a, bh, s); break;
    case 32: launch_dh<32>(a, bh, s); break;
    case 64: launch_dh<64>(a, bh, s); break;
    default: launch_dh<128>(a, bh, s); break;
  }
  return fam_host::check_launch("fam_attention");
}

extern "C" int fam_attention_key_splits(int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t head_dim) {
  if (batch < 1 || heads < 1 || sq < 1 || sk < 1 || head_dim < 1) return 0;
  if (sk <= 256) return 1;
  return (int)std::min<int64_t>(64, (sk + 4 * KB - 1) / (4 * KB));
}

extern "C" int fam_attention_combine(const fam_attn_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_attention_combine: null descriptor");
  FAM_REQUIRE(d->num_splits >= 2 && d->part_o && d->part_ml && d->o, FAM_ERR_INVALID_ARG,
              "fam_attention_combine: needs num_splits >= 2, the partial buffers and o");
  FAM_REQUIRE(d->head_dim % 4 == 0 && d->head_dim >= 8 && d->o_bs % 8 == 0 && d->o_rs % 8 == 0 && d->o_hs % 8 == 0 &&
                  fam_host::aligned16(d->o) && fam_host::aligned16(d->part_o) &&
                  (reinterpret_cast<uintptr_t>(d->part_ml) & 7u) == 0,
              FAM_ERR_INVALID_ARG, "fam_attention_combine: bad head_dim, strides or alignment");
  const int64_t bh = d->batch * d->heads;
  if (bh == 0 || d->sq == 0) return FAM_OK;
  AttnArgs a{};
  a.o = (bf16*)d->o; a.o_bs = d->o_bs; a.o_rs = d->o_rs; a.o_hs = d->o_hs;
  a.H = d->heads; a.Sq = d->sq;
  a.splits = d->num_splits; a.part_o = d->part_o; a.part_ml = d->part_ml;
  const int64_t n = bh * d->sq * (d->head_dim / 4);
  FAM_REQUIRE(n < ((int64_t)1 << 32) - 64 && d->head_dim <= (1 << 20), FAM_ERR_UNSUPPORTED,
              "fam_attention_combine: batch*heads*sq*head_dim/4 must be < 2^32");
  const uint32_t total = (uint32_t)n;
  const int dh = (int)d->head_dim;
  hipStream_t s = (hipStream_t)stream;
  if (a.splits <= 4) launch_combine_s<4>(a, dh, total, s);
  else if (a.splits <= 8) launch_combine_s<8>(a, dh, total, s);
  else if (a.splits <= 16) launch_combine_s<16>(a, dh, total, s);
  else launch_combine_s<0>(a, dh, total, s);
  return fam_host::check_launch("fam_attention_combine");
}

// ---------------------------------------------------------------------------------------
// fam_attention_noalloc: key-split attention (fam_attention + fam_attention_combine) whose split
// partials live in `scratch`, a library-owned device array, instead of caller buffers.  Every
// split writes its partial (o, m, l) for every query it covers, an empty split included (o = 0,
// m = -inf), before the combine reads it, so nothing needs clearing between calls.
#define FAM_ATTN_SCRATCH_BYTES (8u << 20)
static __device__ __align__(256) unsigned char scratch[FAM_ATTN_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device.  In host
// code the array's own name is not a device address; only this pointer may reach a kernel.
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fam_host::set_error("fam_attention_noalloc: no current HIP device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      fam_host::set_error("fam_attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                          hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

// Set-up call: resolves the scratch address on the current device (once per device), so that a
// later fam_attention_noalloc, e.g. one under graph capture, makes no runtime lookup.
extern "C" int64_t fam_attention_noalloc_max_bytes(void) {
  if (scratch_on_current_device() == nullptr) return -(int64_t)FAM_ERR_LAUNCH;
  return (int64_t)FAM_ATTN_SCRATCH_BYTES;
}

extern "C" int fam_attention_noalloc(const fam_attn_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_attention_noalloc: null descriptor");
  FAM_REQUIRE(d->num_splits >= 2 && d->num_splits <= 64, FAM_ERR_INVALID_ARG,
              "fam_attention_noalloc: num_splits must be in [2, 64] (got %d)", d->num_splits);
  FAM_REQUIRE(d->batch >= 0 && d->heads >= 1 && d->sq >= 0 && d->head_dim >= 1, FAM_ERR_INVALID_ARG,
              "fam_attention_noalloc: bad sizes");
  const int64_t rows = (int64_t)d->num_splits * d->batch * d->heads * d->sq;
  const int64_t o_bytes = (rows * d->head_dim * 4 + 255) / 256 * 256;
  const int64_t need = o_bytes + rows * 2 * 4;
  FAM_REQUIRE(need <= (int64_t)FAM_ATTN_SCRATCH_BYTES, FAM_ERR_UNSUPPORTED,
              "fam_attention_noalloc: the split partials need %lld bytes, above the %lld-byte scratch "
              "(num_splits * batch * heads * Sq * (head_dim + 2) * 4 <= %lld)",
              (long long)need, (long long)FAM_ATTN_SCRATCH_BYTES, (long long)FAM_ATTN_SCRATCH_BYTES);
  unsigned char* base = static_cast<unsigned char*>(scratch_on_current_device());
  if (base == nullptr) return FAM_ERR_LAUNCH;
  fam_attn_desc dd = *d;
  dd.part_o = reinterpret_cast<float*>(base);
  dd.part_ml = reinterpret_cast<float*>(base + o_bytes);
  const int rc = fam_attention(&dd, stream);
  if (rc != FAM_OK) return rc;
  if (dd.batch == 0 || dd.sq == 0) return FAM_OK;
  return fam_attention_combine(&dd, stream);
}
