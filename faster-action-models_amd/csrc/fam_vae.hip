// The Wan2.2 VAE encoder's first frame (the policy call's prologue) around the library's GEMM.
// Activations are channels-last rows, one row per pixel ([h*w, C] bf16), so a 1x1 convolution
// is a GEMM over the rows and a 3x3 one is a GEMM over an im2col operand whose row is the
// pixel's 3x3 neighbourhood, taps outermost ((kh*3 + kw)*C + c), zero-padded to a multiple of
// 64 columns.  The kernels here are the non-GEMM steps, each one elementwise pass over the bytes
// it moves (the middle attention's softmax is one wave per row).
#include "fam_common.h"

namespace fam {

// conv1's operand straight from the image: the 2x2 patchify ('b c (h q) (w r) -> b (c r q) h w',
// patched channel c*4 + r*2 + q) fused into the 3x3 im2col of the patched grid (h2 x w2).
// One thread per output element; columns past 9*12 are zero.
__global__ __launch_bounds__(256) void vae_patch_im2col_kernel(const bf16* __restrict__ img, int H, int W,
                                                               bf16* __restrict__ out, int64_t ldo, int kpad,
                                                               int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int h2 = H / 2, w2 = W / 2;
  const int64_t p = i / kpad;
  const int col = (int)(i - p * kpad);
  bf16 v = (bf16)0.0f;
  if (col < 108) {
    const int tap = col / 12, ch = col - tap * 12;
    const int kh = tap / 3, kw = tap - kh * 3;
    const int c = ch >> 2, r = (ch >> 1) & 1, q = ch & 1;
    const int y = (int)(p / w2) + kh - 1, x = (int)(p % w2) + kw - 1;
    if (y >= 0 && y < h2 && x >= 0 && x < w2) v = img[((int64_t)c * H + 2 * y + q) * W + 2 * x + r];
  }
  out[p * ldo + col] = v;
}

// 3x3 im2col of channels-last rows, 8 channels (16 bytes) per thread.  stride 1: 'same' zero
// padding; stride 2: zero padding on the bottom / right only (ZeroPad2d((0, 1, 0, 1)) before a
// stride-2 3x3 convolution), output (H/2) x (W/2).
__global__ __launch_bounds__(256) void im2col3x3_kernel(const bf16* __restrict__ x, int64_t ldx, int H, int W,
                                                        int C, int stride, bf16* __restrict__ out, int64_t ldo,
                                                        int kpad, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int Wo = stride == 1 ? W : W / 2;
  const int k8 = kpad / 8;
  const int64_t p = i / k8;
  const int col = (int)(i - p * k8) * 8;
  bf16x8 v = zero8();
  if (col < 9 * C) {
    const int tap = col / C, c = col - tap * C;
    const int kh = tap / 3, kw = tap - kh * 3;
    const int oy = (int)(p / Wo), ox = (int)(p % Wo);
    const int y = stride == 1 ? oy + kh - 1 : 2 * oy + kh, xx = stride == 1 ? ox + kw - 1 : 2 * ox + kw;
    if (y >= 0 && y < H && xx >= 0 && xx < W) v = load8(x + ((int64_t)y * W + xx) * ldx + c);
  }
  store8(out + p * ldo + col, v);
}

// RMS_norm over the channels of a row (F.normalize: x / max(||x||_2, 1e-12), times sqrt(C) and
// gamma), then the activation; one wave per row, 8 channels per lane and step.
__global__ __launch_bounds__(256) void chan_rmsnorm_kernel(const bf16* __restrict__ x, int64_t ldx, int64_t rows,
                                                           int C, const bf16* __restrict__ gamma, int act,
                                                           bf16* __restrict__ y, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;   // wave-uniform
  const bf16* xr = x + r * ldx;
  float ss = 0.f;
  for (int c = lane * 8; c < C; c += 512) {
    const bf16x8 v = load8(xr + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += to_f(v[e]) * to_f(v[e]);
  }
  ss = wave_sum(ss);
  const float rn = sqrtf((float)C) / fmaxf(sqrtf(ss), 1e-12f);
  for (int c = lane * 8; c < C; c += 512) {
    const bf16x8 v = load8(xr + c), gv = load8(gamma + c);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = to_f(v[e]) * rn * to_f(gv[e]);
      if (act == FAM_ACT_SILU) t = silu(t);
      o[e] = to_bf(t);
    }
    store8(y + r * ldy + c, o);
  }
}

// AvgDown3D of one frame: the frame axis front-padded with ft - 1 zero frames, (t, i, j) blocks
// of ft x fs x fs folded into channels c*F + t*fs*fs + i*fs + j (F = ft*fs*fs), output channel o
// the mean of group [o*G, (o+1)*G), G = Cin*F/Cout; plus `add` (same layout as out) when given.
// One thread per output element.
__global__ __launch_bounds__(256) void vae_avgdown_kernel(const bf16* __restrict__ x, int64_t ldx, int H, int W,
                                                          int Cin, int Cout, int ft, int fs,
                                                          const bf16* __restrict__ add, int64_t ldadd,
                                                          bf16* __restrict__ out, int64_t ldo, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int Wo = W / fs, F = ft * fs * fs, G = Cin * F / Cout;
  const int64_t p = i / Cout;
  const int o = (int)(i - p * Cout);
  const int oy = (int)(p / Wo), ox = (int)(p % Wo);
  float s = 0.f;
  for (int e = o * G; e < (o + 1) * G; ++e) {
    const int c = e / F, rem = e - c * F;
    const int t = rem / (fs * fs), ij = rem - t * fs * fs, ii = ij / fs, jj = ij - ii * fs;
    if (t == ft - 1) s += to_f(x[((int64_t)(oy * fs + ii) * W + ox * fs + jj) * ldx + c]);
  }
  const float a = add ? to_f(add[p * ldadd + o]) : 0.f;
  out[p * ldo + o] = to_bf(s / (float)G + a);
}

// Row softmax of fp32 scores times `scale`, rounded to bf16 (the middle attention's P).
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ s, int64_t lds, int64_t rows,
                                                           int cols, float scale, bf16* __restrict__ p, int64_t ldp) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* sr = s + r * lds;
  const float sl2 = scale * 1.4426950408889634f;
  float m = -INFINITY;
  for (int c = lane; c < cols; c += 64) m = fmaxf(m, sr[c]);
  m = wave_max(m) * sl2;
  float l = 0.f;
  for (int c = lane; c < cols; c += 64) l += __builtin_amdgcn_exp2f(sr[c] * sl2 - m);
  l = wave_sum(l);
  const float inv = 1.0f / l;
  for (int c = lane; c < cols; c += 64) p[r * ldp + c] = to_bf(__builtin_amdgcn_exp2f(sr[c] * sl2 - m) * inv);
}

// out[c, p] = (x[p, c] - mean[c]) * inv_std[c]: the latent normalisation, channels-last rows to
// the channel-first latent.
__global__ __launch_bounds__(256) void chan_affine_nchw_kernel(const bf16* __restrict__ x, int64_t ldx, int64_t P,
                                                               int C, const float* __restrict__ mean,
                                                               const float* __restrict__ inv_std,
                                                               bf16* __restrict__ out, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int c = (int)(i / P);
  const int64_t p = i - (int64_t)c * P;
  out[i] = to_bf((to_f(x[p * ldx + c]) - mean[c]) * inv_std[c]);
}

}  // namespace fam

using namespace fam;

static unsigned blocks_for(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per); }

extern "C" int fam_vae_patch_im2col(const void* img, int64_t H, int64_t W, void* out, int64_t ldo, void* stream) {
  FAM_REQUIRE(img && out, FAM_ERR_INVALID_ARG, "fam_vae_patch_im2col: null pointer");
  FAM_REQUIRE(H >= 2 && W >= 2 && H % 2 == 0 && W % 2 == 0 && H < (1 << 15) && W < (1 << 15) && ldo >= 128,
              FAM_ERR_INVALID_ARG, "fam_vae_patch_im2col: need even H, W (< 32768) and ldo >= 128");
  const int64_t total = (H / 2) * (W / 2) * 128;
  FAM_LAUNCH(vae_patch_im2col_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, (hipStream_t)stream,
             (const bf16*)img, (int)H, (int)W, (bf16*)out, ldo, 128, total);
  return fam_host::check_launch("fam_vae_patch_im2col");
}

extern "C" int fam_im2col3x3(const void* x, int64_t ldx, int64_t H, int64_t W, int64_t C, int64_t stride, void* out,
                             int64_t ldo, int64_t kpad, void* stream) {
  FAM_REQUIRE(x && out, FAM_ERR_INVALID_ARG, "fam_im2col3x3: null pointer");
  FAM_REQUIRE((stride == 1 || (stride == 2 && H % 2 == 0 && W % 2 == 0)) && H >= 1 && W >= 1 && H * W < (1LL << 31),
              FAM_ERR_INVALID_ARG, "fam_im2col3x3: stride 1, or 2 with even H and W");
  FAM_REQUIRE(C >= 8 && C % 8 == 0 && ldx >= C && ldx % 8 == 0 && kpad >= 9 * C && kpad % 8 == 0 && ldo >= kpad &&
                  ldo % 8 == 0 && fam_host::aligned16(x) && fam_host::aligned16(out),
              FAM_ERR_INVALID_ARG, "fam_im2col3x3: C, ldx, kpad (>= 9 C), ldo multiples of 8; 16-byte aligned rows");
  const int64_t P = stride == 1 ? H * W : (H / 2) * (W / 2);
  const int64_t total = P * (kpad / 8);
  FAM_LAUNCH(im2col3x3_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, (hipStream_t)stream, (const bf16*)x, ldx,
             (int)H, (int)W, (int)C, (int)stride, (bf16*)out, ldo, (int)kpad, total);
  return fam_host::check_launch("fam_im2col3x3");
}

extern "C" int fam_chan_rmsnorm(const void* x, int64_t ldx, int64_t rows, int64_t C, const void* gamma, int act,
                                void* y, int64_t ldy, void* stream) {
  FAM_REQUIRE(x && gamma && y, FAM_ERR_INVALID_ARG, "fam_chan_rmsnorm: null pointer");
  FAM_REQUIRE(rows >= 0 && C >= 8 && C % 8 == 0 && ldx >= C && ldy >= C && ldx % 8 == 0 && ldy % 8 == 0 &&
                  fam_host::aligned16(x) && fam_host::aligned16(y) && fam_host::aligned16(gamma),
              FAM_ERR_INVALID_ARG, "fam_chan_rmsnorm: C and strides multiples of 8, 16-byte aligned rows");
  FAM_REQUIRE(act == FAM_ACT_NONE || act == FAM_ACT_SILU, FAM_ERR_INVALID_ARG, "fam_chan_rmsnorm: act none or SiLU");
  if (rows == 0) return FAM_OK;
  FAM_LAUNCH(chan_rmsnorm_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, (hipStream_t)stream, (const bf16*)x, ldx,
             rows, (int)C, (const bf16*)gamma, act, (bf16*)y, ldy);
  return fam_host::check_launch("fam_chan_rmsnorm");
}

extern "C" int fam_vae_avgdown(const void* x, int64_t ldx, int64_t H, int64_t W, int64_t Cin, int64_t Cout,
                               int64_t ft, int64_t fs, const void* add, int64_t ld_add, void* out, int64_t ldo,
                               void* stream) {
  FAM_REQUIRE(x && out, FAM_ERR_INVALID_ARG, "fam_vae_avgdown: null pointer");
  FAM_REQUIRE((ft == 1 || ft == 2) && (fs == 1 || fs == 2) && H % fs == 0 && W % fs == 0 && Cin >= 1 && Cout >= 1 &&
                  (Cin * ft * fs * fs) % Cout == 0 && ldx >= Cin && ldo >= Cout && (!add || ld_add >= Cout) &&
                  H * W < (1LL << 31),
              FAM_ERR_INVALID_ARG, "fam_vae_avgdown: factors 1 or 2 dividing H and W, Cout dividing Cin*ft*fs*fs");
  const int64_t total = (H / fs) * (W / fs) * Cout;
  FAM_LAUNCH(vae_avgdown_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, (hipStream_t)stream, (const bf16*)x,
             ldx, (int)H, (int)W, (int)Cin, (int)Cout, (int)ft, (int)fs, (const bf16*)add, ld_add, (bf16*)out, ldo,
             total);
  return fam_host::check_launch("fam_vae_avgdown");
}

extern "C" int fam_softmax_rows(const float* s, int64_t lds, int64_t rows, int64_t cols, float scale, void* p,
                                int64_t ldp, void* stream) {
  FAM_REQUIRE(s && p, FAM_ERR_INVALID_ARG, "fam_softmax_rows: null pointer");
  FAM_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 30) && lds >= cols && ldp >= cols && scale > 0.f,
              FAM_ERR_INVALID_ARG, "fam_softmax_rows: need cols >= 1, strides >= cols, scale > 0");
  if (rows == 0) return FAM_OK;
  FAM_LAUNCH(softmax_rows_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, (hipStream_t)stream, s, lds, rows,
             (int)cols, scale, (bf16*)p, ldp);
  return fam_host::check_launch("fam_softmax_rows");
}

extern "C" int fam_chan_affine_nchw(const void* x, int64_t ldx, int64_t P, int64_t C, const float* mean,
                                    const float* inv_std, void* out, void* stream) {
  FAM_REQUIRE(x && mean && inv_std && out, FAM_ERR_INVALID_ARG, "fam_chan_affine_nchw: null pointer");
  FAM_REQUIRE(P >= 1 && C >= 1 && ldx >= C && P * C < (1LL << 40), FAM_ERR_INVALID_ARG,
              "fam_chan_affine_nchw: need P, C >= 1 and ldx >= C");
  const int64_t total = P * C;
  FAM_LAUNCH(chan_affine_nchw_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, (hipStream_t)stream, (const bf16*)x,
             ldx, P, (int)C, mean, inv_std, (bf16*)out, total);
  return fam_host::check_launch("fam_chan_affine_nchw");
}
