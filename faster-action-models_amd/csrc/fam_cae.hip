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

// Sum of v over the workgroup (fixed order: wave sums, then waves in order).
__device__ __forceinline__ float cae_block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
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
