// Row quantisation to fp8 (OCP e4m3, the gfx950 convert) with a per-row scale, fused into the
// row operation in front of an fp8 GEMM; and the additive 0 / -inf attention-bias planes of the
// CAE action expert's masks.
//
// Row quantisation (fam_row_q8): one workgroup of 256 lanes per row; each lane keeps its
// J chunks of 8 columns (chunk c = lane + 256 j) in registers, so the row is read once and
// written once.  The row value y is, by mode:
//   ROW         y = x
//   GELU        y = bf16(x / (1 + exp(-1.5957691216057308 (x + 0.044715 x^3))))   (tanh GELU)
//   LN_MOD      y = bf16(bf16(LN(x)) (1 + scale) + shift)
//   ADD_LN_MOD  xo = bf16(x + x2);  y = LN_MOD of xo
// with LN(x) = (x - mean) / sqrt(var + eps), biased variance, fp32 statistics; then
//   a = max |y| over the row,  s[m] = max(a, 1e-12) / 448,  q = fp8(y * (448 / max(a, 1e-12)))
// (448 is e4m3's largest finite value; the convert rounds to nearest even).
#include "fam_common.h"

namespace fam {
namespace {

constexpr int kQ8Threads = 256;
constexpr int kQ8MaxChunks = 8;   // D <= 8 * 8 * 256 = 16384

__device__ __forceinline__ float block_sum4(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();   // red may still be read by the previous reduction
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max4(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float rbf(float v) { return (float)(bf16)v; }

// four fp8 bytes of v[0..3], v clamped to +-448 first (the convert's own range)
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  a = __builtin_amdgcn_fmed3f(a, 448.f, -448.f);
  b = __builtin_amdgcn_fmed3f(b, 448.f, -448.f);
  c = __builtin_amdgcn_fmed3f(c, 448.f, -448.f);
  d = __builtin_amdgcn_fmed3f(d, 448.f, -448.f);
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

template <int MODE, int J>
__global__ __launch_bounds__(kQ8Threads) void row_q8_kernel(const bf16* __restrict__ x, int64_t ldx,
                                                            const bf16* __restrict__ x2, int64_t ldx2,
                                                            const bf16* __restrict__ shift,
                                                            const bf16* __restrict__ scale, float eps,
                                                            uint8_t* __restrict__ y, int64_t ldy,
                                                            float* __restrict__ s, bf16* __restrict__ xo,
                                                            int64_t ldxo, int D) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const int nch = D >> 3;
  float v[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = threadIdx.x + kQ8Threads * j;
    if (c < nch) {
      const bf16x8 a = *(const bf16x8*)(x + m * ldx + 8 * c);
      if (MODE == FAM_Q8_ADD_LN_MOD) {
        const bf16x8 b = *(const bf16x8*)(x2 + m * ldx2 + 8 * c);
        bf16x8 t;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          t[e] = (bf16)((float)a[e] + (float)b[e]);
          v[j][e] = (float)t[e];
        }
        *(bf16x8*)(xo + m * ldxo + 8 * c) = t;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = (float)a[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
    }
  }
  if (MODE == FAM_Q8_LN_MOD || MODE == FAM_Q8_ADD_LN_MOD) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) t += v[j][e];
    const float mean = block_sum4(t, red) / (float)D;
    t = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bool live = threadIdx.x + kQ8Threads * j < nch;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = live ? v[j][e] - mean : 0.f;
        t += d * d;
      }
    }
    const float rstd = 1.f / sqrtf(block_sum4(t, red) / (float)D + eps);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = threadIdx.x + kQ8Threads * j;
      if (c < nch) {
        const bf16x8 sc = *(const bf16x8*)(scale + 8 * c);
        const bf16x8 sh = *(const bf16x8*)(shift + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = rbf(rbf((v[j][e] - mean) * rstd) * (1.f + (float)sc[e]) + (float)sh[e]);
      }
    }
  } else if (MODE == FAM_Q8_GELU) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = v[j][e];
        const float u = 1.5957691216057308f * (a + 0.044715f * a * a * a);
        v[j][e] = rbf(a / (1.f + __expf(-u)));
      }
  }
  float amx = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) amx = fmaxf(amx, fabsf(v[j][e]));   // columns past D hold 0
  amx = fmaxf(block_max4(amx, red), 1e-12f);
  const float mul = 448.f / amx;
  if (threadIdx.x == 0) s[m] = amx * (1.f / 448.f);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = threadIdx.x + kQ8Threads * j;
    if (c < nch) {
      uint2 q;
      q.x = pack_fp8x4(v[j][0] * mul, v[j][1] * mul, v[j][2] * mul, v[j][3] * mul);
      q.y = pack_fp8x4(v[j][4] * mul, v[j][5] * mul, v[j][6] * mul, v[j][7] * mul);
      *(uint2*)(y + m * ldy + 8 * c) = q;
    }
  }
}

// One workgroup per row m < MP of both planes: sb[m, c] = 0 where row m keeps key c of the
// action keys (rows past M keep key 0 only), xb[m, c] = 0 where a real row keeps context key c.
__global__ __launch_bounds__(256) void mask_bias_kernel(const uint8_t* __restrict__ am, const uint8_t* __restrict__ cm,
                                                        int64_t cms, int M, int SK, int NS, int SKP, int NCP,
                                                        float* __restrict__ sb, float* __restrict__ xb) {
  const int m = blockIdx.x;
  const float ninf = -__builtin_inff();
  for (int c = threadIdx.x; c < SKP; c += blockDim.x) {
    const bool keep = m < M ? (c < SK && am[(int64_t)m * SK + c] != 0) : c == 0;
    sb[(int64_t)m * SKP + c] = keep ? 0.f : ninf;
  }
  if (xb != nullptr)
    for (int c = threadIdx.x; c < NCP; c += blockDim.x) {
      const bool keep = m < M && c < NS && cm[(int64_t)m * cms + c] != 0;
      xb[(int64_t)m * NCP + c] = keep ? 0.f : ninf;
    }
}

template <int MODE>
int launch_q8(const fam_rowq8_desc* d, int J, hipStream_t st) {
  const dim3 g((unsigned)d->M), b(kQ8Threads);
#define FAM_Q8_CASE(JJ)                                                                                         \
  case JJ:                                                                                                      \
    FAM_LAUNCH((row_q8_kernel<MODE, JJ>), g, b, 0, st, (const bf16*)d->x, d->ldx, (const bf16*)d->x2, d->ldx2, \
               (const bf16*)d->shift, (const bf16*)d->scale, d->eps, (uint8_t*)d->y, d->ldy, d->s,             \
               (bf16*)d->xo, d->ldxo, (int)d->D);                                                               \
    break;
  switch (J) {
    FAM_Q8_CASE(1) FAM_Q8_CASE(2) FAM_Q8_CASE(3) FAM_Q8_CASE(4)
    FAM_Q8_CASE(5) FAM_Q8_CASE(6) FAM_Q8_CASE(7) FAM_Q8_CASE(8)
  }
#undef FAM_Q8_CASE
  return fam_host::check_launch("fam_row_q8");
}

}  // namespace
}  // namespace fam

using namespace fam;

extern "C" int fam_row_q8(const fam_rowq8_desc* d, void* stream) {
  FAM_REQUIRE(d != nullptr, FAM_ERR_INVALID_ARG, "fam_row_q8: null descriptor");
  FAM_REQUIRE(d->mode >= FAM_Q8_ROW && d->mode <= FAM_Q8_ADD_LN_MOD, FAM_ERR_INVALID_ARG, "fam_row_q8: unknown mode %d",
              d->mode);
  FAM_REQUIRE(d->M >= 0 && d->M < (1LL << 31) && d->D >= 8 && d->D % 8 == 0 &&
                  d->D <= (int64_t)kQ8MaxChunks * 8 * kQ8Threads,
              FAM_ERR_UNSUPPORTED, "fam_row_q8: need 8 <= D <= %d with D a multiple of 8 (D = %lld)",
              kQ8MaxChunks * 8 * kQ8Threads, (long long)d->D);
  FAM_REQUIRE(d->x && d->y && d->s, FAM_ERR_INVALID_ARG, "fam_row_q8: x, y and s are required");
  FAM_REQUIRE(d->ldx >= d->D && d->ldx % 8 == 0 && fam_host::aligned16(d->x) && d->ldy >= d->D && d->ldy % 8 == 0 &&
                  ((uintptr_t)d->y & 7) == 0,
              FAM_ERR_INVALID_ARG, "fam_row_q8: x rows 16-byte aligned, y rows 8-byte aligned, strides >= D");
  const bool ln = d->mode == FAM_Q8_LN_MOD || d->mode == FAM_Q8_ADD_LN_MOD;
  FAM_REQUIRE(!ln || (d->shift && d->scale && fam_host::aligned16(d->shift) && fam_host::aligned16(d->scale)),
              FAM_ERR_INVALID_ARG, "fam_row_q8: the LN modes need 16-byte aligned shift and scale");
  FAM_REQUIRE(!ln || d->eps > 0.f, FAM_ERR_INVALID_ARG, "fam_row_q8: eps must be positive");
  if (d->mode == FAM_Q8_ADD_LN_MOD)
    FAM_REQUIRE(d->x2 && d->xo && d->ldx2 >= d->D && d->ldx2 % 8 == 0 && d->ldxo >= d->D && d->ldxo % 8 == 0 &&
                    fam_host::aligned16(d->x2) && fam_host::aligned16(d->xo),
                FAM_ERR_INVALID_ARG, "fam_row_q8: ADD_LN_MOD needs 16-byte aligned x2 and xo rows");
  if (d->M == 0) return FAM_OK;
  const int J = (int)((d->D / 8 + kQ8Threads - 1) / kQ8Threads);
  const hipStream_t st = (hipStream_t)stream;
  switch (d->mode) {
    case FAM_Q8_ROW: return launch_q8<FAM_Q8_ROW>(d, J, st);
    case FAM_Q8_GELU: return launch_q8<FAM_Q8_GELU>(d, J, st);
    case FAM_Q8_LN_MOD: return launch_q8<FAM_Q8_LN_MOD>(d, J, st);
    default: return launch_q8<FAM_Q8_ADD_LN_MOD>(d, J, st);
  }
}

extern "C" int fam_mask_bias(const uint8_t* am, const uint8_t* cm, int64_t cm_row_stride, int64_t M, int64_t SK,
                             int64_t NS, int64_t MP, int64_t SKP, int64_t NCP, float* sb, float* xb, void* stream) {
  FAM_REQUIRE(am && sb, FAM_ERR_INVALID_ARG, "fam_mask_bias: am and sb are required");
  FAM_REQUIRE(M >= 1 && SK >= 1 && MP >= M && SKP >= SK && MP < (1 << 20) && SKP < (1 << 30) && M * SK < (1LL << 40),
              FAM_ERR_INVALID_ARG, "fam_mask_bias: need 1 <= M <= MP and 1 <= SK <= SKP");
  FAM_REQUIRE(!xb || (cm && NS >= 1 && NCP >= NS && NCP < (1 << 30) && cm_row_stride >= 0 &&
                      (cm_row_stride == 0 || cm_row_stride >= NS)),
              FAM_ERR_INVALID_ARG, "fam_mask_bias: the context plane needs cm, 1 <= NS <= NCP and a row stride of "
                                   "0 or >= NS");
  FAM_LAUNCH(mask_bias_kernel, dim3((unsigned)MP), dim3(256), 0, (hipStream_t)stream, am, cm, cm_row_stride, (int)M,
             (int)SK, (int)NS, (int)SKP, (int)NCP, sb, xb);
  return fam_host::check_launch("fam_mask_bias");
}
