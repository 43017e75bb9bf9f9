// The video expert's token plumbing around its blocks: the patch gather in front of the
// patch-embedding GEMM, the un-patchify scatter after the head GEMM, and a row gather that
// broadcasts a few distinct rows (the per-frame time embedding) to every token.  Each is one
// elementwise pass over the bytes it moves.
#include "fam_common.h"

namespace fam {

// out[b*S + (fi*h + hi)*w + wi, ((c*pt + kt)*ph + kh)*pw + kw] = x[b, c, fi*pt + kt, hi*ph + kh, wi*pw + kw]
__global__ __launch_bounds__(256) void patchify_kernel(const bf16* __restrict__ x, bf16* __restrict__ out,
                                                      int64_t total, int C, int F, int H, int W, int pt, int ph,
                                                      int pw) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int f = F / pt, h = H / ph, w = W / pw, P = C * pt * ph * pw;
  const int64_t row = i / P;
  int col = (int)(i - row * P);
  const int kw = col % pw; col /= pw;
  const int kh = col % ph; col /= ph;
  const int kt = col % pt;
  const int c = col / pt;
  int64_t r = row;
  const int wi = (int)(r % w); r /= w;
  const int hi = (int)(r % h); r /= h;
  const int fi = (int)(r % f);
  const int64_t b = r / f;
  out[i] = x[(((b * C + c) * F + (int64_t)fi * pt + kt) * H + (int64_t)hi * ph + kh) * W + (int64_t)wi * pw + kw];
}

// out[b, c, fi*pt + kt, hi*ph + kh, wi*pw + kw] = y[b*S + (fi*h + hi)*w + wi, ((kt*ph + kh)*pw + kw)*C + c]
__global__ __launch_bounds__(256) void unpatchify_kernel(const bf16* __restrict__ y, bf16* __restrict__ out,
                                                        int64_t total, int C, int f, int h, int w, int pt, int ph,
                                                        int pw) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int Fo = f * pt, Ho = h * ph, Wo = w * pw;
  int64_t r = i;
  const int xo = (int)(r % Wo); r /= Wo;
  const int yo = (int)(r % Ho); r /= Ho;
  const int zo = (int)(r % Fo); r /= Fo;
  const int c = (int)(r % C);
  const int64_t b = r / C;
  const int fi = zo / pt, kt = zo % pt, hi = yo / ph, kh = yo % ph, wi = xo / pw, kw = xo % pw;
  const int64_t row = ((b * f + fi) * h + hi) * w + wi;
  out[i] = y[row * ((int64_t)pt * ph * pw * C) + ((int64_t)(kt * ph + kh) * pw + kw) * C + c];
}

// dst[r, :] = src[idx[r], :], 8 elements per thread; an index outside [0, src_rows) reads the
// nearest valid row (the host cannot see device indices; no access leaves the source)
__global__ __launch_bounds__(256) void gather_rows_kernel(const bf16* __restrict__ src, int64_t lds,
                                                         int64_t src_rows, const int32_t* __restrict__ idx,
                                                         bf16* __restrict__ dst, int64_t ldd, int64_t rows,
                                                         int64_t cols8) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cols8) return;
  const int64_t r = i / cols8, c = (i - r * cols8) * 8;
  const int64_t sr = min(max((int64_t)idx[r], (int64_t)0), src_rows - 1);
  *reinterpret_cast<bf16x8*>(dst + r * ldd + c) = *reinterpret_cast<const bf16x8*>(src + sr * lds + c);
}

}  // namespace fam

using namespace fam;

static bool patch_dims_ok(int64_t B, int64_t C, int64_t F, int64_t H, int64_t W, int64_t pt, int64_t ph,
                          int64_t pw) {
  return B >= 1 && C >= 1 && pt >= 1 && ph >= 1 && pw >= 1 && F >= pt && H >= ph && W >= pw && F % pt == 0 &&
         H % ph == 0 && W % pw == 0 && B * C * F * H * W < (1LL << 38) && C * pt * ph * pw < (1 << 30) &&
         F < (1 << 30) && H < (1 << 30) && W < (1 << 30);
}

extern "C" int fam_patchify(const void* x, int64_t B, int64_t C, int64_t F, int64_t H, int64_t W, int64_t pt,
                            int64_t ph, int64_t pw, void* out, void* stream) {
  FAM_REQUIRE(x && out, FAM_ERR_INVALID_ARG, "fam_patchify: null pointer");
  FAM_REQUIRE(patch_dims_ok(B, C, F, H, W, pt, ph, pw), FAM_ERR_INVALID_ARG,
              "fam_patchify: need positive sizes with F, H, W divisible by the patch (%lld, %lld, %lld)",
              (long long)pt, (long long)ph, (long long)pw);
  const int64_t total = B * C * F * H * W;
  FAM_LAUNCH(patchify_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
             (const bf16*)x, (bf16*)out, total, (int)C, (int)F, (int)H, (int)W, (int)pt, (int)ph, (int)pw);
  return fam_host::check_launch("fam_patchify");
}

extern "C" int fam_unpatchify(const void* y, int64_t B, int64_t C, int64_t f, int64_t h, int64_t w, int64_t pt,
                              int64_t ph, int64_t pw, void* out, void* stream) {
  FAM_REQUIRE(y && out, FAM_ERR_INVALID_ARG, "fam_unpatchify: null pointer");
  FAM_REQUIRE(patch_dims_ok(B, C, f * pt, h * ph, w * pw, pt, ph, pw) && f >= 1 && h >= 1 && w >= 1,
              FAM_ERR_INVALID_ARG, "fam_unpatchify: need positive sizes");
  const int64_t total = B * C * f * pt * h * ph * w * pw;
  FAM_LAUNCH(unpatchify_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
             (const bf16*)y, (bf16*)out, total, (int)C, (int)f, (int)h, (int)w, (int)pt, (int)ph, (int)pw);
  return fam_host::check_launch("fam_unpatchify");
}

extern "C" int fam_gather_rows(const void* src, int64_t ld_src, int64_t src_rows, const int32_t* idx, void* dst,
                               int64_t ld_dst, int64_t rows, int64_t cols, void* stream) {
  FAM_REQUIRE(src && idx && dst, FAM_ERR_INVALID_ARG, "fam_gather_rows: null pointer");
  FAM_REQUIRE(src_rows >= 1 && rows >= 0 && cols >= 8 && cols % 8 == 0 && ld_src >= cols && ld_dst >= cols && ld_src % 8 == 0 &&
                  ld_dst % 8 == 0 && fam_host::aligned16(src) && fam_host::aligned16(dst),
              FAM_ERR_INVALID_ARG, "fam_gather_rows: cols a multiple of 8, strides >= cols and multiples of 8, "
                                   "16-byte aligned rows");
  if (rows == 0) return FAM_OK;
  const int64_t n = rows * (cols / 8);
  FAM_LAUNCH(gather_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
             (const bf16*)src, ld_src, src_rows, idx, (bf16*)dst, ld_dst, rows, cols / 8);
  return fam_host::check_launch("fam_gather_rows");
}
