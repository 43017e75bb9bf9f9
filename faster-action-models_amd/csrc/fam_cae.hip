// Action-VAE decoder of CAE-FastWAM (fp32): latent tokens -> action chunk.
//
//   x = input_proj(z) (+ suite embedding)                     [B, T0, C] -> channels-first [B, C, T0]
//   per stage (stride s): ConvTranspose1d(C, C, 2s, s, s/2) -> GroupNorm(G) -> SiLU
//                         -> x + GN(Conv1d(SiLU(GN(Conv1d(x)))))  (ResidualConv1dBlock, k = 3)
//   crop / zero-pad the time axis to the horizon, output_proj per position -> [B, horizon, A]
//
// One workgroup per (batch row, GroupNorm group): the group's channels over all time steps
// are exactly one GroupNorm reduction, so normalisation needs no cross-workgroup traffic;
// the convolutions read every input channel of the previous stage from the global work
// buffers, so each stage boundary is a kernel boundary.  Fixed-order reductions throughout.
#include "fam_common.h"

namespace fam {

constexpr int CT = 256;  // threads per workgroup

struct CaeArgs {
  int64_t B, T0, L, C, G, T_in, T_out, stride, horizon, A;
  int64_t wchunk;   // input channels per LDS weight chunk of the stage head
  const float* z; const float* suite; const float* in_w; const float* in_b;
  const float* x;   // stage input [B, C, T_in] (stages after the first)
  const float* w; const float* b; const float* gw; const float* gb;
  const float* res; // residual [B, C, T] added after the GroupNorm (or null)
  int silu;
  float* y;         // [B, C, T_out]
  float eps;
  const float* ow; const float* ob; float* out;
};

// Sum of v over the workgroup (fixed order: 16-lane rows by DPP, the four rows by lane swaps,
// then the waves in order).
__device__ __forceinline__ float cae_block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = group4_sum(row16_sum(v));
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// GroupNorm over this workgroup's CG channels x T values held as vals[j] (j-th element of
// this thread, index e = tid + CT*j < n), affine, optional SiLU / residual, store.
template <int NJ>
__device__ __forceinline__ void cae_gn_store(const CaeArgs& a, float (&vals)[NJ], int n, int64_t c0, int64_t T,
                                             float* red) {
  const int tid = threadIdx.x;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) s += (tid + CT * j < n) ? vals[j] : 0.f;
  const float mean = cae_block_sum(s, red) / (float)n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float d = (tid + CT * j < n) ? vals[j] - mean : 0.f;
    q += d * d;
  }
  const float rstd = rsqrtf(cae_block_sum(q, red) / (float)n + a.eps);
  const int64_t bi = blockIdx.x;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = tid + CT * j;
    if (e >= n) continue;
    const int64_t c = c0 + e / T, t = e % T;
    float v = (vals[j] - mean) * rstd * a.gw[c] + a.gb[c];
    if (a.silu) v = v / (1.0f + expf(-v));
    const int64_t o = (bi * a.C + c) * T + t;
    if (a.res) v += a.res[o];
    a.y[o] = v;
  }
}

// Stage head: input projection (first stage) or the previous stage's output, then the
// transposed convolution of this group's channels, GroupNorm, SiLU.  The group's weights
// (w[ci][c0 .. c0 + CG)[0 .. 2s), contiguous per input channel) pass through LDS in chunks of
// `wchunk` input channels after the input rows; every output sums its two taps per input
// channel in input-channel order from the bias.
template <int NJ>
__global__ __launch_bounds__(CT) void cae_up_kernel(CaeArgs a) {
  extern __shared__ float xs[];  // [C][T_in], then [wchunk][CG][2s]
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t bi = blockIdx.x, g = blockIdx.y;
  const int C = (int)a.C, Ti = (int)a.T_in, To = (int)a.T_out, s = (int)a.stride, K = 2 * s, P = s / 2;
  for (int e = tid; e < C * Ti; e += CT) {
    const int c = e / Ti, i = e - c * Ti;
    float v;
    if (a.z) {  // x[c][i] = in_b[c] + sum_l in_w[c][l] z[i][l] (+ suite[c])
      v = a.in_b[c];
      const float* zr = a.z + (bi * a.T0 + i) * a.L;
      for (int64_t l = 0; l < a.L; ++l) v += a.in_w[c * a.L + l] * zr[l];
      if (a.suite) v += a.suite[bi * C + c];
    } else {
      v = a.x[(bi * C + c) * Ti + i];
    }
    xs[e] = v;
  }
  const int CG = C / (int)a.G, c0 = (int)g * CG, CK = CG * K, wc = (int)a.wchunk;
  float* wsm = xs + C * Ti;
  const int n = CG * To;
  float acc[NJ];
  int col[NJ], ihi[NJ], khi[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = tid + CT * j, ee = e < n ? e : 0;
    col[j] = ee / To;
    const int t = ee - col[j] * To;
    // taps: input step i contributes at t = i s - P + kk, kk in [0, 2s): i = ihi (kk = khi) and
    // i = ihi - 1 (kk = khi + s)
    ihi[j] = (t + P) / s;
    khi[j] = t + P - ihi[j] * s;
    acc[j] = a.b[c0 + col[j]];
  }
  for (int ci0 = 0; ci0 < C; ci0 += wc) {
    const int nc = C - ci0 < wc ? C - ci0 : wc;
    __syncthreads();   // the input rows are staged; the previous chunk is consumed
    for (int e = tid; e < nc * CK; e += CT) {
      const int ci = e / CK, r = e - ci * CK;
      wsm[e] = a.w[((int64_t)(ci0 + ci) * C + c0) * K + r];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int hi = ihi[j], lo = hi - 1;
      const float* wr = wsm + col[j] * K;
      for (int ci = 0; ci < nc; ++ci) {
        const float* xr = xs + (ci0 + ci) * Ti;
        if (hi < Ti) acc[j] += xr[hi] * wr[ci * CK + khi[j]];
        if (lo >= 0 && lo < Ti) acc[j] += xr[lo] * wr[ci * CK + khi[j] + s];
      }
    }
  }
  float vals[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) vals[j] = tid + CT * j < n ? acc[j] : 0.f;
  cae_gn_store<NJ>(a, vals, n, c0, To, red);
}

// The stage head on v_mfma_f32_16x16x4f32.  Output step t reads input steps m = (t + P) / s
// (tap r = (t + P) % s) and m - 1 (tap r + s), so the outputs of one residue class r form a GEMM
// D_r[co][m] = sum_q w[ci][co][r + tap s] x[ci][m - tap], q = 2 ci + tap over [0, 2C).  The
// group's weights (w[ci][c0 .. c0 + CG)[0 .. 2s): 2 s CG contiguous floats per input channel)
// pass through LDS in two halves of the input channels by 16-byte loads; the input rows sit
// there with a zero column at each end (steps -1 and T_in); in each half the four waves take
// quarters of the k-steps of every class, and their partial tiles are summed in wave order.
// Requires CG <= 16, s <= 4, at most 16 output steps per class, 2 s CG and C / 2 multiples of 4.
template <int NJ, int S>
__global__ __launch_bounds__(CT) void cae_up_mfma_kernel(CaeArgs a) {
  extern __shared__ float xs[];  // [C][T_in + 2], then [C / 2][CG][2s] weights, then [4][S][64][4]
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int64_t bi = blockIdx.x, g = blockIdx.y;
  const int C = (int)a.C, Ti = (int)a.T_in, To = (int)a.T_out, TP = Ti + 2, P = S / 2, K2 = 2 * S;
  const int CG = C / (int)a.G, c0 = (int)g * CG, RW = CG * K2, CH = C / 2;
  const bool v4 = a.L % 4 == 0;
  for (int e = tid; e < C * TP; e += CT) {
    const int c = e / TP, u = e - c * TP, i = u - 1;
    float v = 0.f;
    if (i >= 0 && i < Ti) {
      if (a.z) {  // x[c][i] = in_b[c] + sum_l in_w[c][l] z[i][l] (+ suite[c])
        v = a.in_b[c];
        const float* zr = a.z + (bi * a.T0 + i) * a.L;
        const float* wr = a.in_w + c * a.L;
        if (v4) {
          for (int64_t l = 0; l < a.L; l += 4) {
            const f32x4 wv = *reinterpret_cast<const f32x4*>(wr + l), zv = *reinterpret_cast<const f32x4*>(zr + l);
            v += wv[0] * zv[0];
            v += wv[1] * zv[1];
            v += wv[2] * zv[2];
            v += wv[3] * zv[3];
          }
        } else {
          for (int64_t l = 0; l < a.L; ++l) v += wr[l] * zr[l];
        }
        if (a.suite) v += a.suite[bi * C + c];
      } else {
        v = a.x[(bi * C + c) * Ti + i];
      }
    }
    xs[e] = v;
  }
  float* wc = xs + C * TP;
  float* part = wc + CH * RW;
  const int nks = CH / 2, ks0 = wave * nks / 4, ks1 = (wave + 1) * nks / 4;   // k-steps of 4 per half
  const int row = l16 < CG ? l16 : 0;
  const float rmask = l16 < CG ? 1.f : 0.f;
  f32x4 acc[S];
  int mcol[S];
  float cmask[S];
#pragma unroll
  for (int r = 0; r < S; ++r) {
    acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    // class r: output steps t = r - P + S m for m in [m0, m1)
    const int m0 = r < P ? 1 : 0, m1 = (To + P - r + S - 1) / S, m = m0 + l16;
    cmask[r] = m < m1 ? 1.f : 0.f;
    mcol[r] = m < m1 ? m : m0;
  }
  for (int h = 0; h < 2; ++h) {
    const int ci0 = h * CH;
    __syncthreads();   // the input rows are staged; the previous half's weights are consumed
    for (int e = tid; e < CH * RW / 4; e += CT) {
      const int ci = e / (RW / 4), q4 = e - ci * (RW / 4);
      *reinterpret_cast<f32x4*>(wc + 4 * e) =
          *reinterpret_cast<const f32x4*>(a.w + ((int64_t)(ci0 + ci) * C + c0) * K2 + 4 * q4);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < S; ++r) {
      for (int ks = ks0; ks < ks1; ++ks) {
        const int q = ks * 4 + lg, ci = q >> 1, tap = q & 1;
        const float av = wc[ci * RW + row * K2 + r + tap * S] * rmask;
        const float bv = xs[(ci0 + ci) * TP + mcol[r] - tap + 1] * cmask[r];
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[r], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < S; ++r) *reinterpret_cast<f32x4*>(part + ((wave * S + r) * 64 + lane) * 4) = acc[r];
  __syncthreads();
  const int n = CG * To;
  float vals[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = tid + CT * j;
    vals[j] = 0.f;
    if (e >= n) continue;
    const int col = e / To, t = e - col * To, r = (t + P) % S, m = (t + P) / S, m0 = r < P ? 1 : 0;
    const int ln = (col >> 2) * 16 + (m - m0), el = col & 3;
    float v = a.b[c0 + col];
#pragma unroll
    for (int w = 0; w < 4; ++w) v += part[((w * S + r) * 64 + ln) * 4 + el];
    vals[j] = v;
  }
  cae_gn_store<NJ>(a, vals, n, c0, To, red);
}

// Conv1d (k = 3, padding 1) of this group's channels over every input channel, GroupNorm,
// then SiLU or the residual add.  The input rows sit in LDS with a zero column at each end (the
// padding), so the three taps need no branch; with WL the group's CG x C x 3 weights are staged
// in LDS too (one contiguous block of the [C][C][3] weight, read once with coalesced loads)
// instead of each output's 3 C scalar global reads.  Every output sums its taps in the order
// (input channel, tap) from the bias.
template <int NJ, bool WL>
__global__ __launch_bounds__(CT) void cae_conv_kernel(CaeArgs a) {
  extern __shared__ float xs[];  // [C][T + 2], then (WL) [CG][C][3]
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t bi = blockIdx.x, g = blockIdx.y;
  const int64_t C = a.C, T = a.T_out, TP = T + 2, CG = C / a.G, c0 = g * CG;
  for (int e = tid; e < (int)(C * TP); e += CT) {
    const int c = e / (int)TP, t = e - c * (int)TP;
    const bool in = t >= 1 && t <= (int)T;
    const float v = a.x[(bi * C + c) * T + (in ? t - 1 : 0)];
    xs[e] = in ? v : 0.f;
  }
  float* wsm = xs + C * TP;
  if constexpr (WL) {
    for (int e = tid; e < (int)(CG * C * 3); e += CT) wsm[e] = a.w[c0 * C * 3 + e];
  }
  __syncthreads();
  const int n = (int)(CG * T);
  float vals[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = tid + CT * j;
    vals[j] = 0.f;
    if (e >= n) continue;
    const int64_t col = e / T, co = c0 + col, t = e % T;
    const float* wr = WL ? wsm + col * C * 3 : a.w + co * C * 3;
    const float* xr = xs + t;   // x[ci][t - 1 + k] at xr[ci (T + 2) + k]
    float acc = a.b[co];
#pragma unroll 4
    for (int64_t ci = 0; ci < C; ++ci) {
      acc += wr[3 * ci] * xr[ci * TP];
      acc += wr[3 * ci + 1] * xr[ci * TP + 1];
      acc += wr[3 * ci + 2] * xr[ci * TP + 2];
    }
    vals[j] = acc;
  }
  cae_gn_store<NJ>(a, vals, n, c0, T, red);
}

// The same convolution on v_mfma_f32_16x16x4f32 (fp32 in and out): D[co][t] = b[co] +
// sum_q W[co][q] X[q / 3][t + q % 3] over q = (input channel, tap) in [0, 3C), W the group's
// CG <= 16 rows of the [C][C][3] weight (contiguous in q; rows past CG read as zero), X the
// zero-padded input rows.  Operand lanes: A[l % 16][q0 + l / 16], B[q0 + l / 16][16 nt + l % 16];
// lane l holds D[4 (l / 16) + r][16 nt + l % 16].  The four waves take consecutive quarters of
// the 3C / 4 k-steps; their partial tiles meet in LDS and are summed in wave order.
template <int NJ, int NT>
__global__ __launch_bounds__(CT) void cae_conv_mfma_kernel(CaeArgs a) {
  extern __shared__ float xs[];  // [C][T + 2], then [CG][3C] weights, then [4][NT][64][4] partials
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, lg = lane >> 4;
  const int64_t bi = blockIdx.x, g = blockIdx.y;
  const int C = (int)a.C, T = (int)a.T_out, TP = T + 2, CG = C / (int)a.G, c0 = (int)g * CG, K3 = 3 * C;
  for (int e = tid; e < C * TP; e += CT) {
    const int c = e / TP, t = e - c * TP;
    const bool in = t >= 1 && t <= T;
    const float v = a.x[(bi * C + c) * T + (in ? t - 1 : 0)];
    xs[e] = in ? v : 0.f;
  }
  float* wsm = xs + C * TP;
  // the group's CG x 3C weights: one contiguous block (16-byte aligned: 3C % 16 == 0 here)
  for (int e = tid; e < CG * K3 / 4; e += CT)
    *reinterpret_cast<f32x4*>(wsm + 4 * e) = *reinterpret_cast<const f32x4*>(a.w + (int64_t)c0 * K3 + 4 * e);
  float* part = wsm + CG * K3;
  __syncthreads();
  const int nks = K3 / 4, ks0 = wave * nks / 4, ks1 = (wave + 1) * nks / 4;
  const int row = l16 < CG ? l16 : 0;
  const float rmask = l16 < CG ? 1.f : 0.f;
  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  int tcol[NT];
  float cmask[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int t = nt * 16 + l16;
    tcol[nt] = t < T ? t : 0;
    cmask[nt] = t < T ? 1.f : 0.f;
  }
  for (int ks = ks0; ks < ks1; ++ks) {
    const int q = ks * 4 + lg, ci = q / 3, k = q - ci * 3;
    const float av = wsm[row * K3 + q] * rmask;
    const float* xr = xs + ci * TP + k;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, xr[tcol[nt]] * cmask[nt], acc[nt], 0, 0, 0);
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    *reinterpret_cast<f32x4*>(part + ((wave * NT + nt) * 64 + lane) * 4) = acc[nt];
  __syncthreads();
  const int n = CG * T;
  float vals[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = tid + CT * j;
    vals[j] = 0.f;
    if (e >= n) continue;
    const int col = e / T, t = e - col * T, nt = t >> 4, ln = (col >> 2) * 16 + (t & 15), r = col & 3;
    float v = a.b[c0 + col];
#pragma unroll
    for (int w = 0; w < 4; ++w) v += part[((w * NT + nt) * 64 + ln) * 4 + r];
    vals[j] = v;
  }
  cae_gn_store<NJ>(a, vals, n, c0, T, red);
}

// output_proj over the horizon (time steps past the decoded length read zeros); the sample's
// decoded rows [C][T_in] and the projection [A][C] are staged in LDS first.
__global__ __launch_bounds__(CT) void cae_out_kernel(CaeArgs a) {
  extern __shared__ float xs[];  // [C][T_in], then ow [A][C]
  const int64_t bi = blockIdx.x;
  const int C = (int)a.C, Ti = (int)a.T_in, A = (int)a.A;
  for (int e = threadIdx.x; e < C * Ti; e += CT) xs[e] = a.x[bi * C * Ti + e];
  float* ow = xs + C * Ti;
  for (int e = threadIdx.x; e < A * C; e += CT) ow[e] = a.ow[e];
  __syncthreads();
  for (int e = threadIdx.x; e < (int)a.horizon * A; e += CT) {
    const int t = e / A, k = e - t * A;
    float acc = a.ob[k];
    if (t < Ti)
      for (int c = 0; c < C; ++c) acc += ow[k * C + c] * xs[c * Ti + t];
    a.out[(bi * a.horizon + t) * A + k] = acc;
  }
}

}  // namespace fam

using namespace fam;

// up: the stage head (LDS: C T_in floats); else the k = 3 convolution (LDS: C (T + 2) floats,
// plus the group's weights where both fit in 64 KB)
static int launch_nj(int n, bool up, const CaeArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)a.B, (unsigned)a.G);
  const int nj = (n + CT - 1) / CT;
  if (nj > 16) return FAM_ERR_UNSUPPORTED;
  const size_t xs = up ? (size_t)(a.C * a.T_in * 4) : (size_t)(a.C * (a.T_out + 2) * 4);
  const size_t wl = (size_t)((a.C / a.G) * a.C * 3 * 4);
  const bool wlds = !up && xs + wl <= 64 * 1024;
  const size_t upl = xs + (size_t)(a.wchunk * (a.C / a.G) * 2 * a.stride * 4);
  // the k = 3 convolution on the matrix cores: a group of <= 16 channels, <= 64 steps, 3C a
  // multiple of 16 (4 waves x k-steps of 4), input rows + weights + partial tiles in 64 KB
  const int64_t CG = a.C / a.G, NT = (a.T_out + 15) / 16;
  const size_t mfl = xs + wl + (size_t)(4 * NT * 64 * 4 * 4);
  // the stage head on the matrix cores: s <= 4, a group of <= 16 channels, <= 16 output steps per
  // residue class, 2C a multiple of 16
  const int64_t st = a.stride, P = st / 2;
  bool up_m = up && st >= 1 && st <= 4 && CG <= 16 && (a.C / 2) % 8 == 0 && (2 * st * CG) % 4 == 0 &&
              ((uintptr_t)a.w & 15u) == 0 &&
              (!a.z || (((uintptr_t)a.in_w & 15u) == 0 && ((uintptr_t)a.z & 15u) == 0));
  for (int64_t r = 0; up_m && r < st; ++r) {
    const int64_t m0 = r < P ? 1 : 0, m1 = (a.T_out + P - r + st - 1) / st;
    up_m = m1 - m0 <= 16;
  }
  const size_t upm = (size_t)((a.C * (a.T_in + 2) + (a.C / 2) * CG * 2 * st + 4 * st * 64 * 4) * 4);
  if (up_m && upm <= 64 * 1024) {
#define FAM_CAE_U(NJ)                                                                       \
    if (nj <= NJ) {                                                                         \
      switch (st) {                                                                         \
        case 1: FAM_LAUNCH((cae_up_mfma_kernel<NJ, 1>), grid, dim3(CT), upm, s, a); break;  \
        case 2: FAM_LAUNCH((cae_up_mfma_kernel<NJ, 2>), grid, dim3(CT), upm, s, a); break;  \
        case 3: FAM_LAUNCH((cae_up_mfma_kernel<NJ, 3>), grid, dim3(CT), upm, s, a); break;  \
        default: FAM_LAUNCH((cae_up_mfma_kernel<NJ, 4>), grid, dim3(CT), upm, s, a); break; \
      }                                                                                     \
      return FAM_OK;                                                                        \
    }
    FAM_CAE_U(2) FAM_CAE_U(4)
#undef FAM_CAE_U
  }
  if (!up && CG <= 16 && NT <= 4 && (3 * a.C) % 16 == 0 && mfl <= 64 * 1024 && ((uintptr_t)a.w & 15u) == 0) {
#define FAM_CAE_M(NJ)                                                                         \
    if (nj <= NJ) {                                                                           \
      switch (NT) {                                                                           \
        case 1: FAM_LAUNCH((cae_conv_mfma_kernel<NJ, 1>), grid, dim3(CT), mfl, s, a); break;  \
        case 2: FAM_LAUNCH((cae_conv_mfma_kernel<NJ, 2>), grid, dim3(CT), mfl, s, a); break;  \
        case 3: FAM_LAUNCH((cae_conv_mfma_kernel<NJ, 3>), grid, dim3(CT), mfl, s, a); break;  \
        default: FAM_LAUNCH((cae_conv_mfma_kernel<NJ, 4>), grid, dim3(CT), mfl, s, a); break; \
      }                                                                                       \
      return FAM_OK;                                                                          \
    }
    FAM_CAE_M(2) FAM_CAE_M(4)
#undef FAM_CAE_M
  }
#define FAM_CAE(NJ)                                                                   \
  if (nj <= NJ) {                                                                     \
    if (up) FAM_LAUNCH((cae_up_kernel<NJ>), grid, dim3(CT), upl, s, a);               \
    else if (wlds) FAM_LAUNCH((cae_conv_kernel<NJ, true>), grid, dim3(CT), xs + wl, s, a); \
    else FAM_LAUNCH((cae_conv_kernel<NJ, false>), grid, dim3(CT), xs, s, a);          \
    return FAM_OK;                                                                    \
  }
  FAM_CAE(2) FAM_CAE(4) FAM_CAE(8) FAM_CAE(16)
#undef FAM_CAE
  return FAM_ERR_UNSUPPORTED;
}

extern "C" int fam_cae_decode(const fam_cae_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_cae_decode: null descriptor");
  FAM_REQUIRE(d->z && d->in_w && d->in_b && d->out_w && d->out_b && d->work && d->out, FAM_ERR_INVALID_ARG,
              "fam_cae_decode: missing tensor pointer");
  FAM_REQUIRE(d->batch >= 0 && d->tokens >= 1 && d->latent_dim >= 1 && d->hidden >= 1 && d->horizon >= 1 &&
                  d->action_dim >= 1 && d->nstages >= 1 && d->nstages <= 3,
              FAM_ERR_INVALID_ARG, "fam_cae_decode: bad sizes");
  const int64_t C = d->hidden, G = C < 8 ? C : 8;
  FAM_REQUIRE(C % G == 0 && C <= 512, FAM_ERR_UNSUPPORTED, "fam_cae_decode: hidden must be <= 512 and divisible by min(8, hidden)");
  int64_t T = d->tokens;
  for (int i = 0; i < d->nstages; ++i) {
    FAM_REQUIRE(d->strides[i] >= 1 && d->up_w[i] && d->up_b[i] && d->gn_w[i] && d->gn_b[i] && d->r1_w[i] &&
                    d->r1_b[i] && d->rg1_w[i] && d->rg1_b[i] && d->r2_w[i] && d->r2_b[i] && d->rg2_w[i] && d->rg2_b[i],
                FAM_ERR_INVALID_ARG, "fam_cae_decode: stage %d incomplete", i);
    FAM_REQUIRE(d->strides[i] <= 64 && (C * T + (C / G) * 2 * d->strides[i]) * 4 <= 64 * 1024, FAM_ERR_UNSUPPORTED,
                "fam_cae_decode: stage %d (stride %lld over %lld steps) does not fit one workgroup's LDS", i,
                (long long)d->strides[i], (long long)T);
    // ConvTranspose1d(k = 2s, stride s, padding s/2): T -> (T-1)s - 2(s/2) + 2s
    T = (T - 1) * d->strides[i] - 2 * (d->strides[i] / 2) + 2 * d->strides[i];
  }
  FAM_REQUIRE((C * T + d->action_dim * C) * 4 <= 64 * 1024, FAM_ERR_UNSUPPORTED,
              "fam_cae_decode: the output projection's rows (%lld x %lld) and weights (%lld x %lld) exceed 64 KiB",
              (long long)C, (long long)T, (long long)d->action_dim, (long long)C);
  FAM_REQUIRE(T <= 1024 && (C / G) * T <= (int64_t)CT * 16 && C * (T + 2) * 4 <= 64 * 1024, FAM_ERR_UNSUPPORTED,
              "fam_cae_decode: decoded length %lld too long for one workgroup per group", (long long)T);
  if (d->batch == 0) return FAM_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t Tmax = T;
  float* wa = d->work;                       // stage head output
  float* wb = d->work + d->batch * C * Tmax;  // residual branch
  float* wr = d->work + 2 * d->batch * C * Tmax;  // stage output
  CaeArgs a{};
  a.B = d->batch; a.T0 = d->tokens; a.L = d->latent_dim; a.C = C; a.G = G; a.horizon = d->horizon; a.A = d->action_dim;
  a.eps = d->gn_eps;
  int64_t Tin = d->tokens;
  for (int i = 0; i < d->nstages; ++i) {
    const int64_t st = d->strides[i];
    const int64_t Tout = (Tin - 1) * st - 2 * (st / 2) + 2 * st;
    // head: (input projection |) transposed conv, GN, SiLU -> wa
    a.z = i == 0 ? d->z : nullptr; a.suite = i == 0 ? d->suite : nullptr; a.in_w = d->in_w; a.in_b = d->in_b;
    a.x = wr; a.T_in = Tin; a.T_out = Tout; a.stride = st;
    a.w = d->up_w[i]; a.b = d->up_b[i]; a.gw = d->gn_w[i]; a.gb = d->gn_b[i]; a.res = nullptr; a.silu = 1; a.y = wa;
    // input channels per weight chunk: what fits in 64 KB beside the input rows (>= 1)
    a.wchunk = std::max<int64_t>(1, std::min<int64_t>(C, (64 * 1024 - C * Tin * 4) / ((C / G) * 2 * st * 4)));
    int rc = launch_nj((int)((C / G) * Tout), true, a, s);
    if (rc) { fam_host::set_error("fam_cae_decode: unsupported stage shape"); return rc; }
    // residual block: conv, GN, SiLU -> wb; conv, GN, + wa -> wr
    a.z = nullptr; a.x = wa; a.T_in = Tout; a.T_out = Tout;
    a.w = d->r1_w[i]; a.b = d->r1_b[i]; a.gw = d->rg1_w[i]; a.gb = d->rg1_b[i]; a.res = nullptr; a.silu = 1; a.y = wb;
    launch_nj((int)((C / G) * Tout), false, a, s);
    a.x = wb; a.w = d->r2_w[i]; a.b = d->r2_b[i]; a.gw = d->rg2_w[i]; a.gb = d->rg2_b[i]; a.res = wa; a.silu = 0; a.y = wr;
    launch_nj((int)((C / G) * Tout), false, a, s);
    Tin = Tout;
  }
  a.x = wr; a.T_in = Tin; a.ow = d->out_w; a.ob = d->out_b; a.out = d->out;
  FAM_LAUNCH(cae_out_kernel, dim3((unsigned)a.B), dim3(CT), (size_t)((C * Tin + d->action_dim * C) * 4), s, a);
  return fam_host::check_launch("fam_cae_decode");
}
