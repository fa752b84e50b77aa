// Shared helpers of the hexkv HIP library: status reporting, 16-byte vector
// type, element conversions and wavefront reductions for gfx950 (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hexkv.h"

namespace hexkv {

// Records a printf-style message for hexkv_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's last error (start of every entry point).
void clear_error();

// Turns a pending launch error into HEXKV_EHIP.
int check_launch(const char *what);

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Reinterpret one 32-bit lane word as a packed pair.  The word is taken by
// value: applying __builtin_bit_cast directly to an ext-vector element
// (v[i]) makes clang read element 0 whatever i is.
__device__ __forceinline__ bf16x2 as_bf16x2(unsigned int w) { return __builtin_bit_cast(bf16x2, w); }
__device__ __forceinline__ f16x2 as_f16x2(unsigned int w) { return __builtin_bit_cast(f16x2, w); }

// ---------------------------------------------------------------- device ---

// Sum over aligned groups of `LPP` consecutive lanes; every lane of a group
// ends with the group's total.  Groups of up to 16 lanes use DPP lane moves
// (quad permutes, then half-row and row mirrors), wider groups ds_bpermute.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LPP >= 1 && LPP <= 64 && (LPP & (LPP - 1)) == 0, "LPP must be a power of two");
  if constexpr (LPP >= 2) v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (LPP >= 4) v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (LPP >= 8) v += dpp_move<0x141>(v);  // row_half_mirror: other quad of 8
  if constexpr (LPP >= 16) v += dpp_move<0x140>(v); // row_mirror: other half of 16
  if constexpr (LPP >= 32) v += __shfl_xor(v, 16);
  if constexpr (LPP >= 64) v += __shfl_xor(v, 32);
  return v;
}

// Butterfly step over lanes l and l ^ OFF (ds_bpermute).
template <int OFF>
__device__ __forceinline__ float xor_sum(float v) {
  return v + __shfl_xor(v, OFF);
}

template <int OFF>
__device__ __forceinline__ float xor_max(float v) {
  return fmaxf(v, __shfl_xor(v, OFF));
}

// xor_sum / xor_max over every offset in [FROM, 64): the total over the
// lanes that agree in their low log2(FROM) bits.
template <int FROM>
__device__ __forceinline__ float sum_from(float v) {
  if constexpr (FROM < 64) return sum_from<FROM * 2>(xor_sum<FROM>(v));
  else return v;
}

template <int FROM>
__device__ __forceinline__ float max_from(float v) {
  if constexpr (FROM < 64) return max_from<FROM * 2>(xor_max<FROM>(v));
  else return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Element traits: 16-byte vector <-> fp32, dot products on packed pairs.
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  static constexpr int kDtype = HEXKV_BF16;
  // dot of the 8 bf16 pairs of a and b, fp32 accumulate (v_dot2c_f32_bf16)
  __device__ __forceinline__ static float dot(u32x4 a, u32x4 b, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a[i]), as_bf16x2(b[i]), acc, false);
    return acc;
  }
  __device__ __forceinline__ static void to_float(u32x4 v, float *f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(v[i] << 16);
      f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static __bf16 from_float(float f) { return static_cast<__bf16>(f); }
};

template <>
struct Elem<_Float16> {
  static constexpr int kDtype = HEXKV_F16;
  __device__ __forceinline__ static float dot(u32x4 a, u32x4 b, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_fdot2(as_f16x2(a[i]), as_f16x2(b[i]), acc, false);
    return acc;
  }
  __device__ __forceinline__ static void to_float(u32x4 v, float *f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2 h = as_f16x2(v[i]);
      f[2 * i] = static_cast<float>(h[0]);
      f[2 * i + 1] = static_cast<float>(h[1]);
    }
  }
  __device__ __forceinline__ static _Float16 from_float(float f) { return static_cast<_Float16>(f); }
};

template <>
struct Elem<float> {
  static constexpr int kDtype = HEXKV_F32;
  __device__ __forceinline__ static float dot(u32x4 a, u32x4 b, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = fmaf(__uint_as_float(a[i]), __uint_as_float(b[i]), acc);
    return acc;
  }
  __device__ __forceinline__ static void to_float(u32x4 v, float *f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  }
  __device__ __forceinline__ static float from_float(float f) { return f; }
};

}  // namespace hexkv
