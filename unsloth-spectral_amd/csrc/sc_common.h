// Shared device/host helpers for the gfx950 spectral kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "spectral_hip.h"

typedef _Float16 h16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- errors
// Thread-local last-error text (host side).
void sc_set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int sc_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define SC_HIP_TRY(expr)                                                         \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess)                                                        \
      return sc_fail(SC_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

static inline int sc_launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sc_fail(SC_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return SC_OK;
}

// ------------------------------------------------------------- wavefront
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Reductions over the four 16-lane rows of a wavefront (lanes n, n+16,
// n+32, n+48): combine the values that MFMA 16x16 outputs spread over rows.
// gfx950's v_permlane32_swap exchanges lanes 32-63 of one register with
// lanes 0-31 of another; applied to two copies of v it leaves (lo, lo) and
// (hi, hi), so op(first, second) holds op(lo, hi) in every lane.  The
// 16-lane variant does the same between odd and even rows.  Both are VALU
// operations (no LDS round trip).
__device__ __forceinline__ float max_over_rows(float v) {
  const uint32_t u = __float_as_uint(v);
  auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(v);
  auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_rows(float v) {
  const uint32_t u = __float_as_uint(v);
  auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t w = __float_as_uint(v);
  auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// Reductions over the four lanes of a quad (lanes 4k .. 4k+3) with DPP
// quad permutes: [1,0,3,2] (0xB1) then [2,3,0,1] (0x4E).
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
}
__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ------------------------------------------------------------ conversions
// Four signed int8 (one dword) -> four exact fp16.  Bias each byte to
// unsigned (b ^ 0x80 = b + 128), splice it under the fp16 exponent pattern
// 0x64 (0x64XX = 1024 + XX), then subtract 1152 with one packed add per pair.
__device__ __forceinline__ half4_t i8x4_to_h4(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const half2_t bias = {(h16)-1152.0f, (h16)-1152.0f};
  half2_t a = __builtin_bit_cast(half2_t, lo) + bias;
  half2_t b = __builtin_bit_cast(half2_t, hi) + bias;
  return (half4_t){a.x, a.y, b.x, b.y};
}
__device__ __forceinline__ half8_t i8x8_to_h8(uint2 w) {
  half4_t a = i8x4_to_h4(w.x), b = i8x4_to_h4(w.y);
  return (half8_t){a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
}

// Scheduling fence for memory instructions: the machine scheduler moves no
// load, store or LDS access across this point, while ALU, MFMA and
// transcendental instructions may still cross it (sched_barrier mask 0x40F).
// Placed right after prefetch loads so that they are issued where the
// source issues them, ahead of the compute they overlap, without keeping
// the surrounding arithmetic from interleaving.
__device__ __forceinline__ void pin_vmem() { __builtin_amdgcn_sched_barrier(0x40F); }

// Value barrier: the compiler cannot look through it, so the value is
// rounded to its own type here.  Used where results must be rounded in the
// reference's order: without it, fptrunc(fmul) and a following add can be
// fused into one (mixed-precision) FMA with a single rounding.
template <class T>
__device__ __forceinline__ T rounded(T x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ half2_t pack_h2(float a, float b) {
  return (half2_t){(h16)a, (h16)b};
}

// ------------------------------------------------------------------ MFMA
// 16x16 outputs: lane l holds D[4*(l/16) + j][l%16], j = 0..3.
// Operand "slots": lane l supplies row/column l%16 and the K-slots of row
// group l/16; A and B use the same slot->k map, so any consistent
// assignment of data to slots yields the sum over k.
__device__ __forceinline__ float4_t mfma_16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4_t mfma_16x16x16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------ XCD mapping
// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx.x % 8).
// Remap so that each XCD walks one contiguous range of work units, keeping
// neighbouring units (shared RoPE rows, shared bases) in one L2.  The grid
// must be xcd_grid(total) wide; returned units >= total are idle.
static inline int xcd_grid(int total) { return ((total + 7) >> 3) << 3; }
__device__ __forceinline__ int xcd_remap(int x, int total) {
  const int per = (total + 7) >> 3;
  const int xcd = x & 7, slot = x >> 3;
  return xcd * per + slot;
}
