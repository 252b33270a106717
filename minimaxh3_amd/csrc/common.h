// Shared helpers for the MI355X (gfx950) FP8 hot-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mxf8.h"

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

namespace mxf8 {

constexpr float kE4m3Max = 448.0f;
constexpr float kScaleFloor = 1.0e-12f;

// ---- error reporting (defined in capi.hip) --------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Compute units of the current device (cached per device; 0 if the query fails).
inline int device_cus() {
  constexpr int kMaxDev = 64;
  static int cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  int n = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    __atomic_store_n(&cache[dev], n, __ATOMIC_RELAXED);
  }
  return n;
}

// ---- scalar conversions ---------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// fp32 -> bf16 bits, round to nearest even (inputs are finite on the hot path; NaN stays NaN)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left free) through the builtin: the compiler's
// own wait insertion takes it into account (it cannot see into inline asm), so it knows
// that no load is in flight after it and adds no wait of its own for one.  The memory
// clobber keeps LDS accesses from moving across it.
__device__ __forceinline__ void wait_vm0() {
  __builtin_amdgcn_s_waitcnt(0x0f70);
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(N) the same way: at most N of this wave's vector memory operations still
// in flight (they complete in issue order).  vmcnt is 6 bits: bits 3:0 and 15:14.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
  asm volatile("" ::: "memory");
}

// Two fp32 values -> two 16-bit values (ODT = MXF8_BF16 / MXF8_F16), a in the low half, in
// one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: round to nearest even, the same bits as
// f32_to_bf16_bits / f32_to_f16_bits for every non-NaN input (NaN stays NaN).
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
template <int ODT>
__device__ __forceinline__ uint32_t cvt_pk_16(float a, float b) {
  const v2f v = {a, b};
  if constexpr (ODT == 0)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2bf));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2h));
}

// Input element loaders: DT = MXF8_BF16 / MXF8_F16 / MXF8_F32.
template <int DT> struct Elem;
template <> struct Elem<MXF8_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float to_f32(T v) { return bf16_bits_to_f32(v); }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};
template <> struct Elem<MXF8_F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float to_f32(T v) { return f16_bits_to_f32(v); }
  static __device__ __forceinline__ float lo(uint32_t w) { return f16_bits_to_f32(w & 0xffffu); }
  static __device__ __forceinline__ float hi(uint32_t w) { return f16_bits_to_f32(w >> 16); }
};
template <> struct Elem<MXF8_F32> {
  typedef float T;
  static __device__ __forceinline__ float to_f32(T v) { return v; }
};

// ---- quantisation arithmetic ----------------------------------------------------------
// scale = max(amax, 1e-12) / 448 with IEEE division (the reference's fp32 semantics).
__device__ __forceinline__ float e4m3_scale(float amax) {
  return __fdiv_rn(fmaxf(amax, kScaleFloor), kE4m3Max);
}

// Correctly rounded x / s given r = RN(1/s): q0 = RN(x r) is faithful, the remainder
// x - s q0 is exact with an fma, and RN(q0 + rem * r) is RN(x / s) (Markstein's
// theorem, binary fp32, no overflow; quotients here are bounded by ~448).  The remainder
// is taken negated, nrem = RN(s q0 - x) = -rem, and the last step is RN(nrem * -r + q0):
// the same value for every x != 0, and for x = -0 the sum -0 + -0 keeps the sign of IEEE
// -0 / s (the positive remainder would give +0).  For s = +inf (a block maximum of inf)
// r is 0: with s capped at the largest finite value in the remainder step, a finite x
// gives +-0 (IEEE x / inf) and +-inf or NaN gives NaN.
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  const float q0 = x * r;
  const float nrem = __builtin_fmaf(q0, fminf(s, 3.40282347e38f), -x);
  return __builtin_fmaf(nrem, -r, q0);
}

__device__ __forceinline__ float clamp448(float q) { return fminf(fmaxf(q, -kE4m3Max), kE4m3Max); }

// Two fp32 values -> two e4m3fn bytes (RNE, hardware conversion) in the low 16 bits.  The
// conversion writes one half of its destination and keeps the other from its last operand;
// a's own bits stand in there (the half is masked off or overwritten), so no zeroed
// register has to be made for it.
__device__ __forceinline__ uint32_t cvt2_e4m3(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false) & 0xffffu;
}
// Four fp32 values -> four e4m3fn bytes packed little-endian in one dword.
__device__ __forceinline__ uint32_t cvt4_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// ---- wave / block reductions ----------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Maximum over a 256-thread block; every thread gets the result.
__device__ __forceinline__ float block256_max(float v, float* red4) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  float r = fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
  __syncthreads();
  return r;
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// LDS tiles with 64- or 128-byte rows are stored as 16-byte chunks, logical chunk c of row
// r at physical chunk c ^ lds_swz(r).  A ds_read_b128 is served 16 lanes at a time over
// 64 four-byte banks (256 bytes); when 16 consecutive rows read the same logical chunk,
// this swizzle puts them on 16 distinct (row within 256 bytes, chunk) bank groups.
template <int ROW_BYTES>
__host__ __device__ constexpr int lds_swz(int row) {
  return (row / (256 / ROW_BYTES)) & (ROW_BYTES / 16 - 1);
}

}  // namespace mxf8
