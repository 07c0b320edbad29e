// Shared pieces of the HIP library: the error channel, host-side argument checks and
// small device helpers (bfloat16 bits, E4M3 conversion, wave reductions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/bux_amd.h"

namespace bux {

// Sets this thread's last error message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears this thread's last error message.
void clear_error();
// Returns BUX_OK, or BUX_E_LAUNCH with the HIP error of the last launch.
int launched(const char* kernel);

#define BUX_CHECK(cond, ...)                                  \
  do {                                                        \
    if (!(cond)) return ::bux::fail(BUX_E_ARGUMENT, __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// --- device helpers --------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float32 -> bfloat16 bits, rounding to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Two float32 -> two bfloat16 (a in the low half), nearest even, by gfx950's
// v_cvt_pk_bf16_f32: the same bits as f32_to_bf16 for every non-NaN value.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(b))) << 16);
}

// Two float32 -> two E4M3 (OCP float8_e4m3fn) codes, nearest even, in the low 16 bits:
// gfx950's v_cvt_pk_fp8_f32. The quantizer only passes values already within +-448.
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

// Four float32 -> four E4M3 codes packed in a word, a in the lowest byte.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// The biased exponent of the least power of two 2^e with 2^e >= q, e clipped to
// [-126, 126]: the reference's _ceil_log2 (precision/blockscaled.py:346-351) of the
// float32 quotient q = amax / 448, from its bits.
__device__ __forceinline__ int scale_exponent(float amax) {
  float q = amax / 448.0f;  // an IEEE division: hipcc rounds float division correctly
  uint32_t bits = __float_as_uint(q);
  int e = static_cast<int>(bits >> 23) + ((bits & 0x7fffffu) != 0u) - 127;
  return e < -126 ? -126 : (e > 126 ? 126 : e);
}

// The same exponent for an amax that is a bfloat16 value (its float32 bits' low 16
// zero), from its bits alone: amax = m 2^E gives E - 8, plus 1 when m > 1.75 (448 =
// 1.75 2^8, and no other 8-bit mantissa puts the quotient within a float32 rounding
// of a power of two, so the division's rounding never moves the result); inf and NaN
// give 126 as the division's bits do. Equal to scale_exponent for every non-negative
// bfloat16 (checked exhaustively).
__device__ __forceinline__ int scale_exponent_bf16(float amax) {
  const uint32_t b = __float_as_uint(amax);
  const int field = static_cast<int>(b >> 23);
  const int e = field - 135 + (((b >> 16) & 0x7fu) > 0x60u ? 1 : 0);
  return field == 255 ? 126 : (e < -126 ? -126 : (e > 126 ? 126 : e));
}

// 2^-e as a float32, exactly, for e in [-126, 126].
__device__ __forceinline__ float power_of_two_down(int e) {
  return __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
}

__device__ __forceinline__ float clip448(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }

// --- the layer's element types ----------------------------------------------------

// A layer computes in its tokens' dtype (the reference's x.dtype, experts/moe.py:846):
// bfloat16, each op's float32 result rounded to it, or float32. Elem<T> moves 8
// elements at once (16 or 32 bytes, aligned) as float32 values and rounds a float32
// result as one op in T does.
template <typename T>
struct Elem;

template <>
struct Elem<uint16_t> {
  static __device__ __forceinline__ void load8(const uint16_t* p, float* v) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
      v[2 * j + 1] = bf16_to_f32(static_cast<uint16_t>(w[j] >> 16));
    }
  }
  static __device__ __forceinline__ void store8(uint16_t* p, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = static_cast<uint32_t>(f32_to_bf16(v[2 * j])) |
             (static_cast<uint32_t>(f32_to_bf16(v[2 * j + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  static __device__ __forceinline__ float value(uint16_t x) { return bf16_to_f32(x); }
  static __device__ __forceinline__ uint16_t make(float x) { return f32_to_bf16(x); }
  static __device__ __forceinline__ float round(float x) { return bf16_to_f32(f32_to_bf16(x)); }
};

template <>
struct Elem<float> {
  static __device__ __forceinline__ void load8(const float* p, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store8(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
  static __device__ __forceinline__ float value(float x) { return x; }
  static __device__ __forceinline__ float make(float x) { return x; }
  static __device__ __forceinline__ float round(float x) { return x; }
};

// --- direct loads into LDS ---------------------------------------------------------

typedef int i32x4 __attribute__((ext_vector_type(4)));

// A raw buffer resource (stride 0) over `bytes` bytes from `base`; offsets past them
// read 0.
__device__ __forceinline__ i32x4 resource(const void* base, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(
      static_cast<int>(bytes > 0xffffffffLL ? 0xffffffffLL : bytes));
  r[3] = 0x00020000;
  return r;
}

// The LDS address of `p` (a location in the workgroup's LDS), as a scalar: the low word
// of a flat pointer into the LDS aperture is the LDS address. (An address-space cast
// would say the same but brings a null check, which hipcc fails to compile in some of
// these kernels.)
__device__ __forceinline__ uint32_t lds_at(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}

// buffer_load_dword{,x4} ... lds: lane i's 4 (16) bytes at the resource's base + voffset +
// soffset land in LDS at M0 + 4 (16) i. Written as inline assembly so that the compiler
// does not track these loads: left to itself it waits for every load in flight
// (vmcnt(0)) before any LDS read that might alias their destinations, which undoes the
// pipeline. The callers count them themselves (s_waitcnt vmcnt).
__device__ __forceinline__ void load_lds16(i32x4 rsrc, uint32_t lds, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset) : "memory", "m0");
}
__device__ __forceinline__ void load_lds4(i32x4 rsrc, uint32_t lds, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset) : "memory", "m0");
}

// load_lds16 where the compiler cannot prove the scalar operands the same in every lane
// (they are): each goes through readfirstlane first.
__device__ __forceinline__ void load_lds16_uniform(i32x4 rsrc, uint32_t lds, int voffset,
                                                   int soffset) {
  const i32x4 r{__builtin_amdgcn_readfirstlane(rsrc[0]), __builtin_amdgcn_readfirstlane(rsrc[1]),
                __builtin_amdgcn_readfirstlane(rsrc[2]), __builtin_amdgcn_readfirstlane(rsrc[3])};
  load_lds16(r, __builtin_amdgcn_readfirstlane(lds), voffset,
             __builtin_amdgcn_readfirstlane(soffset));
}

}  // namespace bux
