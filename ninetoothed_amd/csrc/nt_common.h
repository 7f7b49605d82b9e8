// Shared device helpers for the gfx950 kernels of libnt_mi355x.so.
//
// Element types are carried as raw 16-bit patterns for fp16/bf16 so that loads and
// stores stay plain integer moves; arithmetic always happens in fp32.  Conversions:
//   fp16 <-> fp32 : hardware v_cvt_f16_f32 / v_cvt_f32_f16 through _Float16 (round to
//                   nearest even);
//   bf16 <-> fp32 : bf16 is the top half of an fp32 pattern; fp32 -> bf16 rounds to
//                   nearest even on the discarded 16 bits (quiet NaN kept a NaN).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "nt_mi355x.h"

namespace nt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct f16_t { uint16_t bits; };
struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float f16_bits_to_float(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}
__device__ __forceinline__ uint16_t float_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}
__device__ __forceinline__ float bf16_bits_to_float(uint16_t h) {
  return __builtin_bit_cast(float, ((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Element-type traits: storage type, load-to-float and store-from-float.
template <typename T> struct elem;
template <> struct elem<float> {
  typedef float storage;
  static constexpr int code = NT_DTYPE_F32;
  __device__ __forceinline__ static float to_float(float v) { return v; }
  __device__ __forceinline__ static float from_float(float v) { return v; }
};
template <> struct elem<f16_t> {
  typedef uint16_t storage;
  static constexpr int code = NT_DTYPE_F16;
  __device__ __forceinline__ static float to_float(uint16_t v) { return f16_bits_to_float(v); }
  __device__ __forceinline__ static uint16_t from_float(float v) { return float_to_f16_bits(v); }
};
template <> struct elem<bf16_t> {
  typedef uint16_t storage;
  static constexpr int code = NT_DTYPE_BF16;
  __device__ __forceinline__ static float to_float(uint16_t v) { return bf16_bits_to_float(v); }
  __device__ __forceinline__ static uint16_t from_float(float v) { return float_to_bf16_bits(v); }
};

// Round an fp32 value through a narrower type and back (the application's `.to(dtype)`
// applied to an fp32 accumulator), selected at run time.
__device__ __forceinline__ float round_through(float v, int dtype) {
  if (dtype == NT_DTYPE_F16) return f16_bits_to_float(float_to_f16_bits(v));
  if (dtype == NT_DTYPE_BF16) return bf16_bits_to_float(float_to_bf16_bits(v));
  return v;
}

// Load/store one element of a run-time selected type.
__device__ __forceinline__ float load_as_float(const void* p, int64_t i, int dtype) {
  if (dtype == NT_DTYPE_F32) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  return dtype == NT_DTYPE_F16 ? f16_bits_to_float(h) : bf16_bits_to_float(h);
}
__device__ __forceinline__ void store_from_float(void* p, int64_t i, int dtype, float v) {
  if (dtype == NT_DTYPE_F32) {
    ((float*)p)[i] = v;
  } else if (dtype == NT_DTYPE_F16) {
    ((uint16_t*)p)[i] = float_to_f16_bits(v);
  } else {
    ((uint16_t*)p)[i] = float_to_bf16_bits(v);
  }
}

// Wave64 reductions with cross-lane shuffles.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Lanes of one wave exchanging data through LDS (a lane reads what other lanes wrote): the
// hardware executes a wave's LDS instructions in program order, but the compiler may move
// one lane's load above a store whose address it can prove differs for that lane, which
// lets the load overtake another lane's store.  A call keeps every memory access on its
// side of it.
__device__ __forceinline__ void wave_lds_order() { asm volatile("" ::: "memory"); }

// Compile-time loop: f(std::integral_constant<int, i>) for i in [B, E), so that every
// register index inside f is a constant (used for fixed instruction schedules).
template <int B, int E, typename F>
__host__ __device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

inline bool valid_dtype(int d) { return d == NT_DTYPE_F32 || d == NT_DTYPE_F16 || d == NT_DTYPE_BF16; }
inline bool valid_round(int d) { return d == NT_DTYPE_NONE || d == NT_DTYPE_F16 || d == NT_DTYPE_BF16; }

// Status of the last launch on this thread, as the ABI's int return.
inline int launch_status() { return (int)hipGetLastError(); }

// gemm.hip: a batch of 16-bit products on gemm_dma128_kernel (conv2d's 1 x 1 filters);
// NT_ERR_INVALID, with nothing launched, for a call it does not take; with check_only, 0
// for one it would take, launching nothing either way.
int gemm16_batch128(int dtype, const void* a, int64_t sa_m, int64_t sa_b, const void* b, int64_t sb_k, int64_t sb_b,
                    void* out, int64_t so_m, int64_t so_b, int out_dtype, int64_t M, int64_t N, int64_t K,
                    int64_t batch, int round_dtype, hipStream_t stream, bool check_only = false);

}  // namespace nt
