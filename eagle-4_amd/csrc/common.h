// Shared device helpers of the gfx950 verify kernels: dtype conversion, integer-table loads, lane reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/eagle4_amd.h"

#define E4_DEV __device__ __forceinline__

namespace e4 {

// ---- 16-bit floating point ------------------------------------------------------------------------------------------
// bf16 and fp16 travel as raw uint16 bit patterns; conversions are written out so the rounding is explicit
// (round to nearest even, NaN kept quiet), independent of any compiler intrinsic's mode.

E4_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

E4_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

E4_DEV float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(v);
}

E4_DEV uint16_t f32_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, v);
}

// Type tags: Bf16 / F16 / F32 carry how an element is stored and converted.
struct Bf16 {
  using storage = uint16_t;
  static constexpr int code = EAGLE4_BF16;
  static E4_DEV float load(const storage* p) { return bf16_to_f32(*p); }
  static E4_DEV float to_f32(storage v) { return bf16_to_f32(v); }
  static E4_DEV storage from_f32(float f) { return f32_to_bf16(f); }
};
struct F16 {
  using storage = uint16_t;
  static constexpr int code = EAGLE4_F16;
  static E4_DEV float to_f32(storage v) { return f16_to_f32(v); }
  static E4_DEV storage from_f32(float f) { return f32_to_f16(f); }
};
struct F32 {
  using storage = float;
  static constexpr int code = EAGLE4_F32;
  static E4_DEV float to_f32(storage v) { return v; }
  static E4_DEV storage from_f32(float f) { return f; }
};

// Rounds an fp32 value through a storage dtype (what a store and a reload of that dtype give).
template <typename T>
E4_DEV float round_through(float f) {
  return T::to_f32(T::from_f32(f));
}

// A scalar of a runtime dtype code (0 bf16, 1 f16, 2 f32) as fp32.
E4_DEV float load_scalar(const void* p, int64_t i, int dtype) {
  if (dtype == EAGLE4_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dtype == EAGLE4_F16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

E4_DEV void store_scalar(void* p, int64_t i, int dtype, float f) {
  if (dtype == EAGLE4_BF16)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(f);
  else if (dtype == EAGLE4_F16)
    static_cast<uint16_t*>(p)[i] = f32_to_f16(f);
  else
    static_cast<float*>(p)[i] = f;
}

// Rounds through a runtime dtype code.
E4_DEV float round_code(float f, int dtype) {
  if (dtype == EAGLE4_BF16) return bf16_to_f32(f32_to_bf16(f));
  if (dtype == EAGLE4_F16) return f16_to_f32(f32_to_f16(f));
  return f;
}

// ---- integer tables -----------------------------------------------------------------------------------------------
// Entry (i, j) of an integer table of either dtype, with no branch on the dtype: two dword loads (an int64 entry's
// low and high words, or an int32 entry twice) joined by shifts; for int32, (lo:lo << 32) >> 32 is lo sign-extended.
// Loads of several tables then sit in one basic block and are all in flight before the first wait; behind a branch
// the compiler waits for each table before it issues the next (and a select between the two results is turned back
// into that branch).
E4_DEV int64_t ld(const eagle4_itab& t, int64_t i, int64_t j = 0) {
  const int64_t off = i * t.s0 + j * t.s1;
  const bool wide = t.dtype == EAGLE4_I64;
  const uint32_t* p = static_cast<const uint32_t*>(t.ptr) + (wide ? 2 * off : off);
  const uint32_t lo = p[0], hi = p[wide ? 1 : 0];
  const int sh = wide ? 0 : 32;
  return static_cast<int64_t>(((static_cast<uint64_t>(hi) << 32) | lo) << sh) >> sh;
}

E4_DEV void st(const eagle4_itab& t, int64_t i, int64_t j, int64_t v) {
  const int64_t off = i * t.s0 + j * t.s1;
  if (t.dtype == EAGLE4_I64)
    const_cast<int64_t*>(static_cast<const int64_t*>(t.ptr))[off] = v;
  else
    const_cast<int32_t*>(static_cast<const int32_t*>(t.ptr))[off] = static_cast<int32_t>(v);
}

// ---- lane reductions (wave64) -----------------------------------------------------------------------------------------
// A value of another lane of the same row of 16, through a DPP lane pattern (one VALU operand modifier, no LDS trip).
template <int kCtrl>
E4_DEV float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xF, 0xF, true));
}

// Sum over groups of C adjacent lanes (C a power of two <= 64, all lanes active); every lane of a group gets the same
// bits. Within a row of 16 the partner lanes come by DPP: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1]
// (lane ^ 2), row_half_mirror (the other quad of an 8) and row_mirror (the other 8 of the 16); wider groups use
// ds_bpermute shuffles.
template <int C>
E4_DEV float group_sum(float x) {
  if constexpr (C >= 2) x += dpp<0xB1>(x);
  if constexpr (C >= 4) x += dpp<0x4E>(x);
  if constexpr (C >= 8) x += dpp<0x141>(x);
  if constexpr (C >= 16) x += dpp<0x140>(x);
  if constexpr (C >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (C >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}

template <int C>
E4_DEV float group_max(float x) {
  if constexpr (C >= 2) x = fmaxf(x, dpp<0xB1>(x));
  if constexpr (C >= 4) x = fmaxf(x, dpp<0x4E>(x));
  if constexpr (C >= 8) x = fmaxf(x, dpp<0x141>(x));
  if constexpr (C >= 16) x = fmaxf(x, dpp<0x140>(x));
  if constexpr (C >= 32) x = fmaxf(x, __shfl_xor(x, 16, 64));
  if constexpr (C >= 64) x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

inline int ceil_div(int64_t a, int64_t b) { return static_cast<int>((a + b - 1) / b); }

inline bool is_index_dtype(int d) { return d == EAGLE4_I32 || d == EAGLE4_I64; }
inline bool is_float_dtype(int d) { return d == EAGLE4_BF16 || d == EAGLE4_F16 || d == EAGLE4_F32; }

}  // namespace e4

// Launch-status plumbing of every entry: 0, EAGLE4_NOT_COVERED or the launch's hipError_t.
#define E4_LAUNCH_STATUS() (static_cast<int>(hipGetLastError()))
