// Shared helpers of the hexkv HIP library: status reporting, 16-byte vector
// type, element conversions and wavefront reductions for gfx950 (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "hexkv.h"

namespace hexkv {

// Records a printf-style message for hexkv_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's last error (start of every entry point).
void clear_error();

// Turns a pending launch error into HEXKV_EHIP.
int check_launch(const char *what);

// Devices whose per-device addresses the library caches.
constexpr int kMaxDevices = 64;

// The device `stream` runs on (the current device for the null stream).
int stream_device(hexkv_stream_t stream, int *dev, const char *what);

// Device address of a file-scope __device__ variable on the device that runs
// `stream`, looked up once per device (with that device current) and kept
// in cache[device].  `symbol` is the variable's host-side name, which is not
// a device address itself.
int symbol_address(const void *symbol, std::atomic<void *> *cache, hexkv_stream_t stream, void **addr,
                   const char *what);

// Device address of the status word (HEXKV_STATUS_* bits) of the device that
// runs `stream`.
int status_word(hexkv_stream_t stream, unsigned int **word, const char *what);
// The XCD count of the stream's device (cached per device).
int stream_xcds(hexkv_stream_t stream, int *xcds, const char *what);

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

// Whether a work item read from device memory lies inside a call's
// geometry: row, head group and partition in range, positions
// [first, first + count) within the row's length, the length within
// max_seqlen.  Written without sums that could overflow (first and count are
// checked non-negative first), so an item with extreme values is rejected
// rather than wrapped into range.  Items outside do nothing.
__host__ __device__ inline bool work_item_fits(const hexkv_work_item &it, int rows, int n_groups, int max_parts,
                                               int max_seqlen) {
  return static_cast<unsigned>(it.row) < static_cast<unsigned>(rows) &&
         static_cast<unsigned>(it.head_group) < static_cast<unsigned>(n_groups) &&
         static_cast<unsigned>(it.part) < static_cast<unsigned>(max_parts) && it.parts >= 1 &&
         it.parts <= max_parts && it.first >= 0 && it.count >= 0 && it.len <= max_seqlen &&
         it.count <= it.len - it.first;
}

// ---------------------------------------------------------------- device ---

// Raises status flags (a device-scope atomic OR; `word` may be null).
__device__ __forceinline__ void raise_status(unsigned int *word, unsigned int flags) {
  if (word) atomicOr(word, flags);
}

// The XCD (die) this wave runs on.
__device__ __forceinline__ int xcd_id() {
  int x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 0xf;
}

// Cross-lane reductions, all VALU data movement (no LDS round trip):
// partners within a 16-lane row move by DPP (quad permutes, half-row and row
// mirrors, a row rotation of 8); the two rows of a pair and the two halves
// of the wave are exchanged by gfx950's v_permlane16_swap /
// v_permlane32_swap, which hand each lane its own value and its partner's
// (lane layout pinned on the GPU: swap16(x, x) gives rows (0, 0, 2, 2) and
// (1, 1, 3, 3), swap32(x, x) halves (0, 0) and (1, 1)).  In every step both
// lanes of a pair combine the same two values, so every lane of a group ends
// with bit-identical results.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// The value of lane l ^ OFF (OFF < 16) in lane l.
template <int OFF>
__device__ __forceinline__ float row_partner(float v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8, "offset within a row");
  if constexpr (OFF == 1) return dpp_move<0xB1>(v);  // quad_perm [1,0,3,2]
  else if constexpr (OFF == 2) return dpp_move<0x4E>(v);  // quad_perm [2,3,0,1]
  else if constexpr (OFF == 4) return dpp_move<0x1B>(dpp_move<0x141>(v));  // 7 - l in 8, then l ^ 3 in 4
  else return dpp_move<0x128>(v);  // row_ror:8 = l ^ 8 in 16
}

// op(x, x of lane l ^ OFF) in lane l, for OFF a power of two below 64.
template <int OFF, typename Op>
__device__ __forceinline__ float xor_step(float v, Op op) {
  if constexpr (OFF < 16) {
    return op(v, row_partner<OFF>(v));
  } else {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    unsigned a, b;
    if constexpr (OFF == 16) {
      const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
      a = p[0];
      b = p[1];
    } else {
      static_assert(OFF == 32, "offset");
      const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      a = p[0];
      b = p[1];
    }
    return op(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
  }
}

struct AddOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Sum over aligned groups of `LPP` consecutive lanes; every lane of a group
// ends with the group's total.
template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LPP >= 1 && LPP <= 64 && (LPP & (LPP - 1)) == 0, "LPP must be a power of two");
  if constexpr (LPP >= 2) v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (LPP >= 4) v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (LPP >= 8) v += dpp_move<0x141>(v);  // row_half_mirror: other quad of 8
  if constexpr (LPP >= 16) v += dpp_move<0x140>(v); // row_mirror: other half of 16
  if constexpr (LPP >= 32) v = xor_step<16>(v, AddOp{});
  if constexpr (LPP >= 64) v = xor_step<32>(v, AddOp{});
  return v;
}

// Maximum over aligned groups of `LPP` consecutive lanes; every lane of a
// group ends with the group's maximum.
template <int LPP, int OFF = 1>
__device__ __forceinline__ float group_max(float v) {
  static_assert(LPP >= 1 && LPP <= 64 && (LPP & (LPP - 1)) == 0, "LPP must be a power of two");
  if constexpr (OFF < LPP) return group_max<LPP, OFF * 2>(xor_step<OFF>(v, MaxOp{}));
  else return v;
}

// Total (sum or max) over every offset in [FROM, 64): over the lanes that
// agree in their low log2(FROM) bits.
template <int FROM, typename Op>
__device__ __forceinline__ float reduce_from(float v, Op op) {
  if constexpr (FROM < 64) return reduce_from<FROM * 2>(xor_step<FROM>(v, op), op);
  else return v;
}

template <int FROM>
__device__ __forceinline__ float sum_from(float v) {
  return reduce_from<FROM>(v, AddOp{});
}

template <int FROM>
__device__ __forceinline__ float max_from(float v) {
  return reduce_from<FROM>(v, MaxOp{});
}

__device__ __forceinline__ float wave_max(float v) { return max_from<1>(v); }

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
