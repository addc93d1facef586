// Shared helpers for the gfx950 kernels and the C ABI: vector types, error
// reporting, 16-bit float conversions and wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <type_traits>

#include "../../include/diffucore_amd.h"

namespace dc {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- errors

void set_error(const char* fmt, ...);
void clear_error();

inline int fail(int code, const char* msg) {
  set_error("%s", msg);
  return code;
}

// Checks the launch that was just enqueued.
inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return DC_EHIP;
  }
  return DC_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline int elem_bytes(int dtype) {
  switch (dtype) {
    case DC_F16: case DC_BF16: return 2;
    case DC_F32: case DC_I32: return 4;
    default: return 0;
  }
}

// ---------------------------------------------------------------- 16-bit floats

// bits of a 16-bit float -> float32 (exact)
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

// float32 -> 16-bit float bits, round to nearest even (IEEE conversions)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  __bf16 b = (__bf16)x;
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  _Float16 h = (_Float16)x;
  return __builtin_bit_cast(uint16_t, h);
}

template <int DT>
__device__ __forceinline__ float h16_to_f32(uint32_t bits16) {
  if constexpr (DT == DC_BF16) return bf16_to_f32(bits16);
  else return f16_to_f32(bits16);
}
template <int DT>
__device__ __forceinline__ uint32_t f32_to_h16(float x) {
  if constexpr (DT == DC_BF16) return f32_to_bf16_bits(x);
  else return f32_to_f16_bits(x);
}

// Pins a float32 value in a register. Without it the backend folds
// "fp32 multiply/add, then convert to fp16" into one v_fma_mix*_f16, which
// rounds the exact result once; the reference rounds to float32 first.
__device__ __forceinline__ float materialize(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Round a float32 to the output dtype and back (for the double-rounded bias add).
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == DC_F32) return x;
  else return h16_to_f32<DT>(f32_to_h16<DT>(x));
}

// ---------------------------------------------------------------- compile-time loops

// static_for<N>(f) calls f(std::integral_constant<int, i>{}) for i = 0 .. N-1.
// Array indices inside f are constants from the start, so small register
// arrays are promoted to registers before loop unrolling would run.
template <int I, int N>
struct StaticFor {
  template <class F>
  __device__ __forceinline__ static void run(F& f) {
    f(std::integral_constant<int, I>{});
    StaticFor<I + 1, N>::run(f);
  }
};
template <int N>
struct StaticFor<N, N> {
  template <class F>
  __device__ __forceinline__ static void run(F&) {}
};
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  StaticFor<0, N>::run(f);
}

// ---------------------------------------------------------------- wave reductions

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

}  // namespace dc
