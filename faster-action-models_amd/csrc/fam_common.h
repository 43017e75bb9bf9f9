// Shared device helpers for the gfx950 kernels of the action-DiT hot path.
//
// Conventions used by every kernel in this library:
//   * storage is bf16 (`__bf16`), arithmetic is fp32; `(__bf16)f` lowers to the
//     hardware round-to-nearest-even convert (v_cvt_pk_bf16_f32) on gfx950;
//   * a wavefront is 64 lanes; reductions use cross-lane shuffles, never atomics;
//   * 16-byte vector loads (8 x bf16) need 16-byte aligned rows, which the host
//     validation layer checks before any launch.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fam_hip.h"

namespace fam {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

__device__ __forceinline__ float to_f(bf16 v) { return (float)v; }
__device__ __forceinline__ bf16 to_bf(float v) { return (bf16)v; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Lane l's value and lane (l ^ 16)'s / (l ^ 32)'s, lower lane first, through the gfx950 lane
// swaps (VALU, no LDS round trip as __shfl_xor's ds_bpermute): for a commutative op, r[0] op r[1]
// is the same in both lanes of a pair and equals v op __shfl_xor(v, 16 / 32).
__device__ __forceinline__ void pair_xor16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair_xor32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  float a, b;
  pair_xor32(v, a, b);
  return a + b;
}
__device__ __forceinline__ float max_xor32(float v) {
  float a, b;
  pair_xor32(v, a, b);
  return fmaxf(a, b);
}

// Sum over the four lane groups {l, l^16, l^32, l^48} (MFMA 16x16 column reductions); the same
// pairing and order as v += shfl_xor(v, 16); v += shfl_xor(v, 32).
__device__ __forceinline__ float group4_sum(float v) {
  float a, b;
  pair_xor16(v, a, b);
  return sum_xor32(a + b);
}
__device__ __forceinline__ float group4_max(float v) {
  float a, b;
  pair_xor16(v, a, b);
  return max_xor32(fmaxf(a, b));
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// Sum over the 16 lanes of a row, the same in every lane: the pairs of the xor butterfly 1, 2,
// 4, 8 through DPP (quad_perm [1,0,3,2], [2,3,0,1]; row_half_mirror pairs the two equal quads of
// each half-row, row_mirror the two equal half-rows), so the result equals the __shfl_xor loop.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return v;
}

// Sum over the 64 lanes, the same in every lane, without LDS: the 16-lane rows (DPP), then the
// four rows (lane swaps).  (wave_sum's order is the reverse: 32, 16, ..., 1.)
__device__ __forceinline__ float wave_sum_valu(float v) { return group4_sum(row16_sum(v)); }

__device__ __forceinline__ bf16x8 load8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ void store8(bf16* p, bf16x8 v) { *reinterpret_cast<bf16x8*>(p) = v; }

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
  return z;
}

// Branch-free guarded 16-byte load: a lane whose element is out of range reads `safe` (any
// valid address of the same tensor) and gets zeros.  Keeping the load unconditional lets
// the compiler batch it with its neighbours instead of wrapping each one in an exec-masked
// branch.
__device__ __forceinline__ bf16x8 load8_if(bool ok, const bf16* p, const bf16* safe) {
  const bf16x8 v = load8(ok ? p : safe);
  return ok ? v : zero8();
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), evaluated as x / (1 + e^(-2u)) (the
  // same function: 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u))) with the hardware exp2 and reciprocal,
  // branch-free (the library tanhf runs two divergent paths) and without the cancellation of
  // 1 + tanh(u) for negative u; e^(-2u) overflowing to +inf gives x * 0
  const float k0 = 0.7978845608028654f;
  const float u = k0 * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(u * -2.8853900817779268f);   // e^(-2u) = 2^(-2u log2 e)
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// 0.5 x (1 + erf(x / sqrt(2))): nn.GELU() without approximation (the Cosmos backbone's
// FeedForward, activation_fn "gelu"), with the device library's erff
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f)); }

// x sigmoid(x) with the hardware exp2 and reciprocal (no IEEE division); e^(-x) overflowing to
// +inf gives x * 0
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// MFMA 16x16x32 bf16 -> fp32 (gfx950).  Lane l holds A[row=l%16][k=8*(l/16)..+7],
// B[k=8*(l/16)..+7][col=l%16]; D[row=4*(l/16)+i][col=l%16], i = 0..3.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// MFMA 32x32x16 bf16 -> fp32 (gfx950).  Lane l holds A[row=l%32][k=8*(l/32)..+7],
// B[k=8*(l/32)..+7][col=l%32]; D register r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Workgroup barrier that waits for this wave's LDS operations only (lgkmcnt(0)), not for its
// global loads: __syncthreads() also drains vmcnt, which would stall on register prefetches
// issued just before it.  The empty asm statements keep the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);   // vmcnt 63 (no wait), expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Raw buffer resource over [base, base + bytes): loads at byte offsets >= bytes return 0.
// The descriptor lives in SGPRs, so `base` and `bytes` must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
// 16 bytes at byte offset voff (per lane) + soff (wave-uniform).  Only voff is range-checked
// against the descriptor: an offset that must read zero past the end goes into voff.
__device__ __forceinline__ bf16x8 buffer_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return __builtin_bit_cast(bf16x8, v);
}

}  // namespace fam

// Host-side helpers shared by the C-ABI wrappers.
namespace fam_host {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// Compute units of the device current at the first call (cached; 256, MI355X's count, when the
// query fails); the launch plans size their grids with it.
inline int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus = n;
  }
  return cus;
}
// Launch-timing events armed by fam_set_launch_events (null: plain launches).
extern thread_local hipEvent_t t_evt_start, t_evt_stop;
}  // namespace fam_host

// Every kernel launch of the library goes through this macro: when the calling thread has
// armed a start/stop event pair, the first launch records the start at its begin and every
// launch the stop at its end (hipExtLaunchKernelGGL), so the pair spans the kernels of one
// library call; this is how bench.py measures per-call kernel durations.
#define FAM_LAUNCH(kernel, grid, block, shmem, stream, ...)                                              \
  do {                                                                                                   \
    if (fam_host::t_evt_stop != nullptr) {                                                               \
      /* a call of several launches: the first records the start, every one the stop */                 \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, fam_host::t_evt_start, fam_host::t_evt_stop, \
                            0, __VA_ARGS__);                                                             \
      fam_host::t_evt_start = nullptr;                                                                   \
    } else                                                                                               \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                               \
  } while (0)

#define FAM_REQUIRE(cond, code, ...)            \
  do {                                          \
    if (!(cond)) {                              \
      fam_host::set_error(__VA_ARGS__);         \
      return (code);                            \
    }                                           \
  } while (0)
