// Error plumbing of the C ABI and the small elementwise kernels of the denoise loop:
// the flow-matching Euler update, the sinusoidal timestep embedding, the per-block
// modulation add and the small-K linear of the action encoder.
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "fam_common.h"

namespace fam_host {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

thread_local hipEvent_t t_evt_start = nullptr, t_evt_stop = nullptr;

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return FAM_ERR_LAUNCH;
  }
  return FAM_OK;
}

}  // namespace fam_host

extern "C" int fam_set_launch_events(void* start_event, void* stop_event) {
  FAM_REQUIRE((start_event == nullptr) == (stop_event == nullptr), FAM_ERR_INVALID_ARG,
              "fam_set_launch_events: give both events or neither");
  fam_host::t_evt_start = (hipEvent_t)start_event;
  fam_host::t_evt_stop = (hipEvent_t)stop_event;
  return FAM_OK;
}

namespace fam {

// out = bf16(sample + bf16(model_output * delta)): the two roundings of the eager
// `sample + model_output * delta` in bf16 (SCH:88).
__global__ __launch_bounds__(256) void euler_kernel(const bf16* x, const bf16* __restrict__ v,
                                                    const bf16* __restrict__ delta, bf16* out, int64_t n,
                                                    int64_t inner) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x);
  if (i >= n) return;
  const float d = to_f(delta[i / inner]);
  out[i] = to_bf(to_f(x[i]) + to_f(to_bf(to_f(v[i]) * d)));
}

// Vector form: 8 elements per 16-byte chunk, EU chunks per thread (chunk t + 256 j of the
// workgroup's block), all loads issued before the arithmetic.  Needs n % 8 == 0, inner % 8 == 0
// and 16-byte aligned pointers, so the 8 elements of a chunk share one delta.
template <int EU>
__global__ __launch_bounds__(256) void euler_vec_kernel(const bf16* x, const bf16* __restrict__ v,
                                                        const bf16* __restrict__ delta, bf16* out, int64_t n8,
                                                        int64_t inner8) {
  const int64_t base = (int64_t)blockIdx.x * (256 * EU) + threadIdx.x;
  bf16x8 xv[EU], vv[EU];
  float dv[EU];
#pragma unroll
  for (int j = 0; j < EU; ++j) {
    const int64_t c = base + 256 * j, cc = c < n8 ? c : 0;
    xv[j] = load8(x + cc * 8);
    vv[j] = load8(v + cc * 8);
    dv[j] = to_f(delta[(uint32_t)cc / (uint32_t)inner8]);   // n8 < 2^31 (host check)
  }
#pragma unroll
  for (int j = 0; j < EU; ++j) {
    const int64_t c = base + 256 * j;
    if (c >= n8) continue;
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf(to_f(xv[j][e]) + to_f(to_bf(to_f(vv[j][e]) * dv[j])));
    store8(out + c * 8, o);
  }
}

// out[t, i] = cos/sin(p_t * 10000^(-i/half)) in fp64, rounded to bf16.
__global__ __launch_bounds__(256) void sinusoid_kernel(const bf16* __restrict__ pos, bf16* __restrict__ out,
                                                       int64_t T, int64_t dim) {
  const int64_t half = dim / 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= T * half) return;
  const int64_t t = idx / half, i = idx - t * half;
  const double p = (double)to_f(pos[t]);
  const double f = pow(10000.0, -(double)i / (double)half);
  const double a = p * f;
  out[t * dim + i] = to_bf((float)cos(a));
  out[t * dim + half + i] = to_bf((float)sin(a));
}

// out[t, l, :] = bf16(mod[l, :] + tmod[t, :]); one thread per 8 elements.
__global__ __launch_bounds__(256) void add_mod_kernel(const bf16* __restrict__ tmod, const bf16* __restrict__ mod,
                                                      bf16* __restrict__ out, int64_t T, int64_t L, int64_t n) {
  const int64_t n8 = n / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= T * L * n8) return;
  const int64_t c = (idx % n8) * 8;
  const int64_t tl = idx / n8;
  const int64_t l = tl % L, t = tl / L;
  bf16x8 a = load8(tmod + t * n + c), b = load8(mod + l * n + c), o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf(to_f(a[e]) + to_f(b[e]));
  store8(out + (t * L + l) * n + c, o);
}

// y[m, n] = sum_k x[m, k] w[n, k] + b[n], one thread per output, K <= 64.
template <typename XT>
__global__ __launch_bounds__(256) void linear_smallk_kernel(const XT* __restrict__ x, int64_t ldx,
                                                            const bf16* __restrict__ w, const bf16* __restrict__ b,
                                                            bf16* __restrict__ y, int64_t ldy, int64_t M, int64_t N,
                                                            int64_t K) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx - m * N;
  float acc = 0.f;
  for (int64_t k = 0; k < K; ++k) acc += (float)x[m * ldx + k] * to_f(w[n * K + k]);
  if (b) acc += to_f(b[n]);
  y[m * ldy + n] = to_bf(acc);
}

// y = bf16(act(x)) elementwise over rows of 8-element chunks; one thread per chunk.
__global__ __launch_bounds__(256) void act_rows_kernel(const bf16* x, int64_t ldx, bf16* y, int64_t ldy,
                                                       uint32_t rows, uint32_t c8, int act) {
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  if (idx >= rows * c8) return;
  const uint32_t r = idx / c8, c = (idx - r * c8) * 8;
  const bf16x8 v = load8(x + (int64_t)r * ldx + c);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = to_f(v[e]);
    o[e] = to_bf(act == FAM_ACT_SILU ? silu(f) : act == FAM_ACT_GELU_TANH ? gelu_tanh(f)
                 : act == FAM_ACT_GELU_ERF ? gelu_erf(f) : act == FAM_ACT_RELU ? fmaxf(f, 0.f) : f);
  }
  store8(y + (int64_t)r * ldy + c, o);
}

}  // namespace fam

using namespace fam;

extern "C" int fam_version(void) { return FAM_ABI_VERSION; }

extern "C" int fam_act_rows(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows,
                            int64_t cols, int act, void* stream) {
  FAM_REQUIRE(x && y, FAM_ERR_INVALID_ARG, "fam_act_rows: x and y must be non-null");
  FAM_REQUIRE(act >= FAM_ACT_NONE && act <= FAM_ACT_GELU_ERF, FAM_ERR_INVALID_ARG, "fam_act_rows: unknown act %d", act);
  FAM_REQUIRE(rows >= 0 && cols >= 0 && cols % 8 == 0 && x_row_stride % 8 == 0 && y_row_stride % 8 == 0 &&
                  x_row_stride >= cols && y_row_stride >= cols,
              FAM_ERR_INVALID_ARG, "fam_act_rows: cols and row strides must be multiples of 8, strides >= cols");
  FAM_REQUIRE(fam_host::aligned16(x) && fam_host::aligned16(y), FAM_ERR_INVALID_ARG,
              "fam_act_rows: x and y must be 16-byte aligned");
  const int64_t n = rows * (cols / 8);
  FAM_REQUIRE(n < ((int64_t)1 << 32) - 256, FAM_ERR_UNSUPPORTED, "fam_act_rows: too many elements");
  if (n == 0) return FAM_OK;
  FAM_LAUNCH(act_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, (const bf16*)x,
             x_row_stride, (bf16*)y, y_row_stride, (uint32_t)rows, (uint32_t)(cols / 8), act);
  return fam_host::check_launch("fam_act_rows");
}

extern "C" const char* fam_last_error(void) { return fam_host::g_err; }

static unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

extern "C" int fam_euler_step(const void* sample, const void* model_output, const void* delta, void* out,
                              int64_t n, int64_t inner, void* stream) {
  FAM_REQUIRE(sample && model_output && delta && out, FAM_ERR_INVALID_ARG, "fam_euler_step: null pointer");
  FAM_REQUIRE(n >= 0 && inner >= 1, FAM_ERR_INVALID_ARG, "fam_euler_step: need n >= 0 and inner >= 1");
  if (n == 0) return FAM_OK;
  if (n % 8 == 0 && inner % 8 == 0 && n / 8 < ((int64_t)1 << 31) && fam_host::aligned16(sample) &&
      fam_host::aligned16(model_output) && fam_host::aligned16(out)) {
    const int64_t n8 = n / 8;
    FAM_LAUNCH(euler_vec_kernel<4>, dim3((unsigned)((n8 + 1023) / 1024)), dim3(256), 0, (hipStream_t)stream,
               (const bf16*)sample, (const bf16*)model_output, (const bf16*)delta, (bf16*)out, n8, inner / 8);
    return fam_host::check_launch("fam_euler_step");
  }
  FAM_LAUNCH(euler_kernel, dim3(blocks_for(n)), dim3(256), 0, (hipStream_t)stream, (const bf16*)sample,
                     (const bf16*)model_output, (const bf16*)delta, (bf16*)out, n, inner);
  return fam_host::check_launch("fam_euler_step");
}

extern "C" int fam_sinusoid(const void* positions, void* out, int64_t T, int64_t dim, void* stream) {
  FAM_REQUIRE(positions && out, FAM_ERR_INVALID_ARG, "fam_sinusoid: null pointer");
  FAM_REQUIRE(T >= 0 && dim >= 2 && dim % 2 == 0, FAM_ERR_INVALID_ARG, "fam_sinusoid: dim must be even and >= 2");
  if (T == 0) return FAM_OK;
  FAM_LAUNCH(sinusoid_kernel, dim3(blocks_for(T * (dim / 2))), dim3(256), 0, (hipStream_t)stream,
                     (const bf16*)positions, (bf16*)out, T, dim);
  return fam_host::check_launch("fam_sinusoid");
}

extern "C" int fam_add_modulation(const void* t_mod, const void* modulation, void* out, int64_t T, int64_t L,
                                  int64_t n, void* stream) {
  FAM_REQUIRE(t_mod && modulation && out, FAM_ERR_INVALID_ARG, "fam_add_modulation: null pointer");
  FAM_REQUIRE(T >= 0 && L >= 0 && n > 0 && n % 8 == 0, FAM_ERR_INVALID_ARG, "fam_add_modulation: n must be a positive multiple of 8");
  FAM_REQUIRE(fam_host::aligned16(t_mod) && fam_host::aligned16(modulation) && fam_host::aligned16(out),
              FAM_ERR_INVALID_ARG, "fam_add_modulation: pointers must be 16-byte aligned");
  if (T == 0 || L == 0) return FAM_OK;
  FAM_LAUNCH(add_mod_kernel, dim3(blocks_for(T * L * (n / 8))), dim3(256), 0, (hipStream_t)stream,
                     (const bf16*)t_mod, (const bf16*)modulation, (bf16*)out, T, L, n);
  return fam_host::check_launch("fam_add_modulation");
}

extern "C" int fam_linear_smallk(const void* x, int64_t ldx, int x_f32, const void* w, const void* b, void* y,
                                 int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  FAM_REQUIRE(x && w && y, FAM_ERR_INVALID_ARG, "fam_linear_smallk: null pointer");
  FAM_REQUIRE(M >= 0 && N >= 1 && K >= 1 && K <= 64, FAM_ERR_INVALID_ARG, "fam_linear_smallk: need 1 <= K <= 64");
  FAM_REQUIRE(ldx >= K && ldy >= N, FAM_ERR_INVALID_ARG, "fam_linear_smallk: bad leading dimensions");
  if (M == 0) return FAM_OK;
  if (x_f32)
    FAM_LAUNCH(linear_smallk_kernel<float>, dim3(blocks_for(M * N)), dim3(256), 0, (hipStream_t)stream,
                       (const float*)x, ldx, (const bf16*)w, (const bf16*)b, (bf16*)y, ldy, M, N, K);
  else
    FAM_LAUNCH(linear_smallk_kernel<bf16>, dim3(blocks_for(M * N)), dim3(256), 0, (hipStream_t)stream,
                       (const bf16*)x, ldx, (const bf16*)w, (const bf16*)b, (bf16*)y, ldy, M, N, K);
  return fam_host::check_launch("fam_linear_smallk");
}
