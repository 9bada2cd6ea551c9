// Shared device/host helpers for the limn HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/limn_hip.h"

namespace limn {

typedef unsigned short u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef u16 u16x8 __attribute__((ext_vector_type(8)));
typedef u16 u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ---- storage <-> compute conversions --------------------------------------------------------
// bfloat16 and float16 are storage widths: they are widened to float to compute and rounded
// (round to nearest even) once on store.

__device__ __forceinline__ float bf16_to_f32(u16 bits) { return __uint_as_float(((unsigned)bits) << 16); }

__device__ __forceinline__ u16 f32_to_bf16(float x) {
  __bf16 h = (__bf16)x;  // RNE; NaN stays NaN
  return __builtin_bit_cast(u16, h);
}

__device__ __forceinline__ float f16_to_f32(u16 bits) { return (float)__builtin_bit_cast(_Float16, bits); }

__device__ __forceinline__ u16 f32_to_f16(float x) { return __builtin_bit_cast(u16, (_Float16)x); }

// Element type tags: what lives in memory (Storage) and what arithmetic runs in (Compute).
struct F64 {
  typedef double Storage;
  typedef double Compute;
  static __device__ __forceinline__ double load(const double* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(double* p, int64_t i, double v) { p[i] = v; }
};
struct F32 {
  typedef float Storage;
  typedef float Compute;
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
struct BF16 {
  typedef u16 Storage;
  typedef float Compute;
  static __device__ __forceinline__ float load(const u16* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ void store(u16* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
  static __device__ __forceinline__ u16 pack(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ float unpack(u16 v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ f32x16 mfma32(u16x8 a, u16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // two floats rounded into one 32-bit word, the first in the low half (v_cvt_pk_bf16_f32)
  static __device__ __forceinline__ unsigned pack2(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
  }
};
struct F16 {
  typedef u16 Storage;
  typedef float Compute;
  static __device__ __forceinline__ float load(const u16* p, int64_t i) { return f16_to_f32(p[i]); }
  static __device__ __forceinline__ void store(u16* p, int64_t i, float v) { p[i] = f32_to_f16(v); }
  static __device__ __forceinline__ u16 pack(float v) { return f32_to_f16(v); }
  static __device__ __forceinline__ float unpack(u16 v) { return f16_to_f32(v); }
  static __device__ __forceinline__ f32x16 mfma32(u16x8 a, u16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ unsigned pack2(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, f16x2));
  }
};

// Items base .. base+7 of an accumulator, rounded to the storage width and packed in order: the
// 16-byte MFMA operand they form.
template <typename T>
__device__ __forceinline__ u16x8 pack8(const f32x16& s, int base) {
  const u32x4 w = {T::pack2(s[base], s[base + 1]), T::pack2(s[base + 2], s[base + 3]), T::pack2(s[base + 4], s[base + 5]),
                   T::pack2(s[base + 6], s[base + 7])};
  return __builtin_bit_cast(u16x8, w);
}

// The width row statistics (L, delta) are kept at: float for the half widths, else the dtype.
template <typename T>
struct Stat {
  typedef typename T::Compute type;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ double fast_exp2(double x) { return exp2(x); }

}  // namespace limn

// ---- host-side error reporting --------------------------------------------------------------
namespace limn {
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_hip(hipError_t err, const char* doing);
}  // namespace limn
