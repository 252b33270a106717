// Dynamic e4m3 quantizers (HBM-bound): per-row activations/weights and the attention
// Q / K / V quantizers.  One pass over the input wherever the statistic is local to
// the tile (rows, 128-row blocks); the per-channel V scale and the key mean need a
// reduction over the whole sequence first (a partial-reduction kernel writes one
// [chunk][D] slab per workgroup into the caller's workspace and the consumer folds the
// slabs in a fixed order, so results do not depend on scheduling).
#include <stdarg.h>

#include <atomic>
#include <mutex>

#include "common.h"
#include "rowq.h"

namespace mxf8 {

// ---------------------------------------------------------------------------------------
// quantize_rows: kernels/fp8_linear.py:8-24 (per row: amax -> scale -> codes)
// ---------------------------------------------------------------------------------------

// Fast path: one wave per row, the whole row held in registers as NC 16-byte chunks per
// lane (chunk c of lane l covers elements [(c*64 + l) * E, +E)).  Requires K % E == 0
// and 16-byte aligned rows.  All of the row's loads are issued before the first use (a
// loop that folds each chunk into the max as it arrives measured 3-19% slower).
//
// The row maximum compares absolute-value bit patterns as integers (two 16-bit ones per
// v_pk_max_u16): for every non-NaN value the order of |x| is the order of its pattern
// with the sign cleared, and NaN patterns lie above inf's.  A row whose largest pattern is
// a NaN takes the float maximum instead, which skips NaN as the reference's tl.max does.
// The codes are then made and stored chunk by chunk.
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

template <int DT>
struct RowBits;
template <>
struct RowBits<MXF8_BF16> {
  static constexpr uint32_t kInf = 0x7f80u;
  static __device__ __forceinline__ float to_f32(uint32_t b) { return bf16_bits_to_f32(b); }
};
template <>
struct RowBits<MXF8_F16> {
  static constexpr uint32_t kInf = 0x7c00u;
  static __device__ __forceinline__ float to_f32(uint32_t b) { return f16_bits_to_f32(b); }
};
template <>
struct RowBits<MXF8_F32> {
  static constexpr uint32_t kInf = 0x7f800000u;
  static __device__ __forceinline__ float to_f32(uint32_t b) { return __uint_as_float(b); }
};

// Largest |x| pattern of this lane's chunks.
template <int DT, int NC>
__device__ __forceinline__ uint32_t chunk_absmax_bits(const uint4 (&v)[NC]) {
  if constexpr (DT == MXF8_F32) {
    uint32_t m = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) m = max(m, w[i] & 0x7fffffffu);
    }
    return m;
  } else {
    v2u16 m = {0, 0};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(v2u16, w[i] & 0x7fff7fffu));
    }
    return max((uint32_t)m[0], (uint32_t)m[1]);
  }
}

// Largest |x| pattern of this lane's chunks with NaN skipped (for rows that hold a NaN).
// Integer work only: float conversions here would be shared with the code loop's and
// held in registers across the maximum.
template <int DT, int NC>
__device__ __forceinline__ uint32_t chunk_absmax_bits_nonan(const uint4 (&v)[NC]) {
  constexpr uint32_t kInf = RowBits<DT>::kInf;
  uint32_t m = 0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == MXF8_F32) {
        const uint32_t b = w[i] & 0x7fffffffu;
        m = max(m, b <= kInf ? b : 0u);
      } else {
        const uint32_t b0 = w[i] & 0x7fffu, b1 = (w[i] >> 16) & 0x7fffu;
        m = max(m, max(b0 <= kInf ? b0 : 0u, b1 <= kInf ? b1 : 0u));
      }
    }
  }
  return m;
}

// The e4m3 codes of one chunk (E elements) at orow + idx * E.
template <int DT>
__device__ __forceinline__ void chunk_store_codes(const uint4& q, int64_t idx, float s, float r,
                                                  uint8_t* __restrict__ orow) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if constexpr (DT == MXF8_F32) {
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = clamp448(div_by_scale(__uint_as_float(w[i]), s, r));
    *reinterpret_cast<uint32_t*>(orow + idx * 4) = cvt4_e4m3(f[0], f[1], f[2], f[3]);
  } else {
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = clamp448(div_by_scale(Elem<DT>::lo(w[i]), s, r));
      f[2 * i + 1] = clamp448(div_by_scale(Elem<DT>::hi(w[i]), s, r));
    }
    *reinterpret_cast<uint2*>(orow + idx * 8) = make_uint2(cvt4_e4m3(f[0], f[1], f[2], f[3]),
                                                           cvt4_e4m3(f[4], f[5], f[6], f[7]));
  }
}

// FULL: every lane's NC chunks lie inside the row (K = NC * 64 * E), so no chunk is tested.
// Waves per SIMD asked of the register allocator for whole bf16 rows (the row takes 4 NC
// registers; without a target the scheduler spends registers on early conversions, down
// to two waves at NC = 24).  The other variants keep the allocator's choice, which a
// target this tight would turn into spills.
template <int DT, int NC, bool FULL>
constexpr int quant_rows_waves() {
  if (DT != MXF8_BF16 || !FULL) return 1;
  return NC <= 8 ? 8 : NC <= 12 ? 6 : NC <= 16 ? 5 : NC <= 24 ? 4 : 3;
}

template <int DT, int NC, bool FULL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(quant_rows_waves<DT, NC, FULL>())))
void quant_rows_reg_kernel(const void* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t ldx, uint8_t* __restrict__ x8,
                                                             float* __restrict__ scale) {
  typedef typename Elem<DT>::T T;
  constexpr int E = 16 / sizeof(T);
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const T*>(x) + row * ldx);
  const int64_t nchunk = K / E;
  uint4 v[NC];
  if constexpr (FULL) {
#pragma unroll
    for (int c = 0; c < NC; ++c) v[c] = xr[c * 64 + lane];
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)c * 64 + lane;
      v[c] = idx < nchunk ? xr[idx] : make_uint4(0, 0, 0, 0);
    }
  }
  uint32_t mb = chunk_absmax_bits<DT, NC>(v);
  if (__builtin_amdgcn_ballot_w64(mb > RowBits<DT>::kInf)) mb = chunk_absmax_bits_nonan<DT, NC>(v);
  const float amax = wave_max(RowBits<DT>::to_f32(mb));
  const float s = e4m3_scale(amax);
  const float r = __fdiv_rn(1.0f, s);
  uint8_t* orow = x8 + row * K;
  if constexpr (FULL) {
#pragma unroll
    for (int c = 0; c < NC; ++c) chunk_store_codes<DT>(v[c], c * 64 + lane, s, r, orow);
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)c * 64 + lane;
      if (idx < nchunk) chunk_store_codes<DT>(v[c], idx, s, r, orow);
    }
  }
  if (lane == 0) scale[row] = s;
}

// General path (any K, any alignment): one 256-thread block per row, two passes.
template <int DT>
__global__ __launch_bounds__(256) void quant_rows_generic_kernel(const void* __restrict__ x, int64_t M,
                                                                 int64_t K, int64_t ldx,
                                                                 uint8_t* __restrict__ x8,
                                                                 float* __restrict__ scale) {
  typedef typename Elem<DT>::T T;
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = static_cast<const T*>(x) + row * ldx;
  float amax = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(Elem<DT>::to_f32(xr[k])));
  amax = block256_max(amax, red);
  const float s = e4m3_scale(amax);
  const float r = __fdiv_rn(1.0f, s);
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float q = clamp448(div_by_scale(Elem<DT>::to_f32(xr[k]), s, r));
    x8[row * K + k] = (uint8_t)(cvt2_e4m3(q, 0.0f) & 0xff);
  }
  if (threadIdx.x == 0) scale[row] = s;
}

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

template <int DT, int NC>
static void launch_quant_rows_reg(const void* x, int64_t M, int64_t K, int64_t ldx, uint8_t* x8, float* scale,
                                  hipStream_t st) {
  const dim3 grid((unsigned)cdiv(M, 4));
  if (K == (int64_t)NC * 64 * (16 / (DT == MXF8_F32 ? 4 : 2)))
    quant_rows_reg_kernel<DT, NC, true><<<grid, dim3(256), 0, st>>>(x, M, K, ldx, x8, scale);
  else
    quant_rows_reg_kernel<DT, NC, false><<<grid, dim3(256), 0, st>>>(x, M, K, ldx, x8, scale);
}

template <int DT>
static int quant_rows_dispatch(const void* x, int64_t M, int64_t K, int64_t ldx, uint8_t* x8, float* scale,
                               hipStream_t st) {
  typedef typename Elem<DT>::T T;
  constexpr int E = 16 / sizeof(T);
  const bool aligned = (K % E == 0) && (ldx % E == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)x8 % 16 == 0);
  const int64_t nchunk = K / E;
  const int64_t per_lane = cdiv(nchunk, 64);
  if (aligned && per_lane <= 32 && cdiv(M, 4) <= 0x7fffffff) {
    switch (per_lane <= 1 ? 1 : per_lane <= 2 ? 2 : per_lane <= 4 ? 4 : per_lane <= 6 ? 6 : per_lane <= 8 ? 8
            : per_lane <= 12 ? 12 : per_lane <= 16 ? 16 : per_lane <= 24 ? 24 : 32) {
      case 1: launch_quant_rows_reg<DT, 1>(x, M, K, ldx, x8, scale, st); break;
      case 2: launch_quant_rows_reg<DT, 2>(x, M, K, ldx, x8, scale, st); break;
      case 4: launch_quant_rows_reg<DT, 4>(x, M, K, ldx, x8, scale, st); break;
      case 6: launch_quant_rows_reg<DT, 6>(x, M, K, ldx, x8, scale, st); break;
      case 8: launch_quant_rows_reg<DT, 8>(x, M, K, ldx, x8, scale, st); break;
      case 12: launch_quant_rows_reg<DT, 12>(x, M, K, ldx, x8, scale, st); break;
      case 16: launch_quant_rows_reg<DT, 16>(x, M, K, ldx, x8, scale, st); break;
      case 24: launch_quant_rows_reg<DT, 24>(x, M, K, ldx, x8, scale, st); break;
      default: launch_quant_rows_reg<DT, 32>(x, M, K, ldx, x8, scale, st); break;
    }
  } else {
    if (M > 0x7fffffff) return set_error(MXF8_EINVAL, "quant_rows: M=%lld too large for the general path", (long long)M);
    quant_rows_generic_kernel<DT><<<dim3((unsigned)M), dim3(256), 0, st>>>(x, M, K, ldx, x8, scale);
  }
  return check_launch("quant_rows");
}

// ---------------------------------------------------------------------------------------
// adaLN modulation fused with the per-row quantizer.  The DiT block's input to the QKV and
// MLP-up linears is y = LN(x) * (1 + scale_b) + shift_b (LayerNorm without affine, the
// adaLN shift / scale of the row's batch item b), which FP8Linear.forward then
// quantizes per row (kernels/fp8_linear.py:27-42).  Here one pass reads x once and writes
// the e4m3 codes and row scales of y (and, optionally, y itself in bf16).
//   LN: fp32 mean and biased variance of the row, rstd = 1 / sqrt(var + eps),
//       n = (x - mean) * rstd
//   EAGER = false: y = bf16(n * (1 + scale) + shift) in fp32, one rounding (the fused
//                  pointwise code of a compiled block)
//   EAGER = true:  torch's eager bf16 op sequence, a rounding after each op:
//                  n -> bf16, (1 + scale) -> bf16, product -> bf16, sum -> bf16
// One wave per row with the row in registers (NC 16-byte chunks per lane).
// ---------------------------------------------------------------------------------------
template <int NC, bool EAGER, bool WRITE_Y>
__global__ __launch_bounds__(256) void adaln_quant_rows_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t C,
                                                               int64_t ldx, int64_t S,
                                                               const uint16_t* __restrict__ shift,
                                                               const uint16_t* __restrict__ scale, int64_t ldm,
                                                               float eps, uint8_t* __restrict__ x8,
                                                               float* __restrict__ sa, uint16_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t b = row / S;
  const int64_t nchunk = C / 8;
  uint4 v[NC];
  row_load_bf16<NC>(x + row * ldx, nchunk, lane, v);
  float amax = adaln_modulate_bf16<NC, EAGER>(v, C, nchunk, lane, reinterpret_cast<const uint4*>(shift + b * ldm),
                                               reinterpret_cast<const uint4*>(scale + b * ldm), eps);
  if constexpr (WRITE_Y) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)c * 64 + lane;
      // non-temporal: at 720p the rows (477 MB) exceed the MALL and the LoRA down-projection
      // reads them next; streamed out early, they leave it fewer write-backs to wait on (the
      // pair 329 -> 312 us on MI355X)
      if (idx < nchunk)
        __builtin_nontemporal_store(v4i{(int)v[c].x, (int)v[c].y, (int)v[c].z, (int)v[c].w},
                                    reinterpret_cast<v4i*>(y + row * C) + idx);
    }
  }
  amax = wave_max(amax);
  const float s = e4m3_scale(amax);
  row_store_codes_bf16<NC>(v, nchunk, lane, s, __fdiv_rn(1.0f, s), x8 + row * C);
  if (lane == 0) sa[row] = s;
}

template <int NC, bool EAGER>
static void launch_adaln(const uint16_t* x, int64_t M, int64_t C, int64_t ldx, int64_t S, const uint16_t* sh,
                         const uint16_t* sc, int64_t ldm, float eps, uint8_t* x8, float* sa, uint16_t* y,
                         hipStream_t st) {
  const dim3 grid((unsigned)cdiv(M, 4));
  if (y)
    adaln_quant_rows_kernel<NC, EAGER, true><<<grid, 256, 0, st>>>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y);
  else
    adaln_quant_rows_kernel<NC, EAGER, false><<<grid, 256, 0, st>>>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y);
}

template <bool EAGER>
static void adaln_dispatch(int nc, const uint16_t* x, int64_t M, int64_t C, int64_t ldx, int64_t S,
                           const uint16_t* sh, const uint16_t* sc, int64_t ldm, float eps, uint8_t* x8, float* sa,
                           uint16_t* y, hipStream_t st) {
  switch (nc) {
    case 1: launch_adaln<1, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
    case 2: launch_adaln<2, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
    case 4: launch_adaln<4, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
    case 6: launch_adaln<6, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
    case 8: launch_adaln<8, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
    case 12: launch_adaln<12, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
    default: launch_adaln<16, EAGER>(x, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y, st); break;
  }
}

// ---------------------------------------------------------------------------------------
// Attention quantizers (kernels/fp8_attention.py:39-170)
// ---------------------------------------------------------------------------------------

struct Strides4 {
  int64_t b, h, s, d;
};

// Loads 8 consecutive-in-d elements of row `s` as fp32.  VEC: d contiguous and the
// 8-element group 16-byte aligned; otherwise element-wise strided loads.
// Raw form of load8 for the vector case: the 16 bytes of 8 consecutive-in-d elements of
// row s (issued early, converted with cvt8 later, so several loads are in flight at once).
template <int DT>
__device__ __forceinline__ uint4 raw8(const void* base, const Strides4& st, int64_t s, int d0) {
  typedef typename Elem<DT>::T T;
  return *reinterpret_cast<const uint4*>(static_cast<const T*>(base) + s * st.s + d0);
}
template <int DT>
__device__ __forceinline__ void cvt8(const uint4& v, float f[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = Elem<DT>::lo(w[i]);
    f[2 * i + 1] = Elem<DT>::hi(w[i]);
  }
}

template <int DT, bool VEC>
__device__ __forceinline__ void load8(const void* base, const Strides4& st, int64_t s, int d0, float f[8]) {
  typedef typename Elem<DT>::T T;
  const T* p = static_cast<const T*>(base) + s * st.s + (int64_t)d0 * st.d;
  if constexpr (VEC) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = Elem<DT>::lo(w[i]);
      f[2 * i + 1] = Elem<DT>::hi(w[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = Elem<DT>::to_f32(p[(int64_t)i * st.d]);
  }
}

// Q (IS_K = false) and K (IS_K = true) quantizer of one (128-row block blk, b*H + h) tile
// by a 256-thread block (nblk blocks per head; red: 4 floats of LDS).  Thread t handles
// the 8-wide d-chunk (t % CPR) of rows (t / CPR) + RPP * p.
template <int DT, int D, bool IS_K, bool VEC>
__device__ __forceinline__ void quant_qk_tile(const void* __restrict__ src, const Strides4& st, int64_t H, int64_t S,
                                              int64_t Sp, float c, const float* __restrict__ mean,
                                              uint8_t* __restrict__ out8, float* __restrict__ scale_out, int64_t blk,
                                              int64_t bh, int64_t nblk, float* red) {
  constexpr int CPR = D / 8;      // chunks per row
  constexpr int RPP = 256 / CPR;  // rows per pass
  constexpr int NP = 128 / RPP;   // passes
  const int64_t b = bh / H, h = bh % H;
  const void* base = static_cast<const char*>(src) + (b * st.b + h * st.h) * (int64_t)sizeof(typename Elem<DT>::T);
  const int cc = threadIdx.x % CPR;
  const int rl = threadIdx.x / CPR;
  float mu[8];
  if constexpr (IS_K) {
#pragma unroll
    for (int i = 0; i < 8; ++i) mu[i] = mean[bh * D + cc * 8 + i];
  }
  float f[NP][8];
  float amax = 0.0f;
  uint4 raw[VEC ? NP : 1];
  if constexpr (VEC) {
    // every pass's load in flight before the first use
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int64_t s = blk * 128 + rl + RPP * p;
      raw[p] = s < S ? raw8<DT>(base, st, s, cc * 8) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t s = blk * 128 + rl + RPP * p;
    if (s < S) {
      if constexpr (VEC)
        cvt8<DT>(raw[p], f[p]);
      else
        load8<DT, VEC>(base, st, s, cc * 8, f[p]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[p][i] = IS_K ? (f[p][i] - mu[i]) : (f[p][i] * c);
        amax = fmaxf(amax, fabsf(f[p][i]));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[p][i] = 0.0f;
    }
  }
  amax = block256_max(amax, red);
  const float sc = e4m3_scale(amax);
  const float r = __fdiv_rn(1.0f, sc);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t s = blk * 128 + rl + RPP * p;  // rows in [S, Sp) are written as zeros
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = clamp448(div_by_scale(f[p][i], sc, r));
    uint2 o;
    o.x = cvt4_e4m3(q[0], q[1], q[2], q[3]);
    o.y = cvt4_e4m3(q[4], q[5], q[6], q[7]);
    *reinterpret_cast<uint2*>(out8 + (bh * Sp + s) * D + cc * 8) = o;
  }
  if (threadIdx.x == 0) scale_out[bh * nblk + blk] = sc;
}

// One block per (128-row block, b*H + h).
template <int DT, int D, bool IS_K, bool VEC>
__global__ __launch_bounds__(256) void attn_quant_qk_kernel(const void* __restrict__ src, Strides4 st, int64_t H,
                                                            int64_t S, int64_t Sp, float c,
                                                            const float* __restrict__ mean,
                                                            uint8_t* __restrict__ out8,
                                                            float* __restrict__ scale_out) {
  __shared__ float red[4];
  quant_qk_tile<DT, D, IS_K, VEC>(src, st, H, S, Sp, c, mean, out8, scale_out, blockIdx.x, blockIdx.y, gridDim.x,
                                  red);
}

// Partial column reductions over a chunk of rows: SUM (key mean) or ABSMAX (V scale).
// grid (nch, B*H); writes part[bh][chunk][d].
template <int DT, int D, bool ABSMAX, bool VEC>
__global__ __launch_bounds__(256) void attn_colreduce_kernel(const void* __restrict__ src, Strides4 st, int64_t H,
                                                             int64_t S, int64_t rows_per_chunk,
                                                             float* __restrict__ part) {
  constexpr int CPR = D / 8;
  constexpr int RPP = 256 / CPR;
  __shared__ float red[RPP][D + 1];
  const int64_t ch = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / H, h = bh % H;
  const void* base = static_cast<const char*>(src) + (b * st.b + h * st.h) * (int64_t)sizeof(typename Elem<DT>::T);
  const int cc = threadIdx.x % CPR;
  const int rl = threadIdx.x / CPR;
  const int64_t r0 = ch * rows_per_chunk;
  const int64_t r1 = min(S, r0 + rows_per_chunk);
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  int64_t s = r0 + rl;
  if constexpr (VEC) {
    // 8 rows' loads in flight together; rows are folded in the same order as one at a time
    constexpr int U = 8;
    for (; s + (U - 1) * RPP < r1; s += U * RPP) {
      uint4 raw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) raw[u] = raw8<DT>(base, st, s + u * RPP, cc * 8);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float f[8];
        cvt8<DT>(raw[u], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = ABSMAX ? fmaxf(acc[i], fabsf(f[i])) : acc[i] + f[i];
      }
    }
  }
  for (; s < r1; s += RPP) {
    float f[8];
    load8<DT, VEC>(base, st, s, cc * 8, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = ABSMAX ? fmaxf(acc[i], fabsf(f[i])) : acc[i] + f[i];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[rl][cc * 8 + i] = acc[i];
  __syncthreads();
  if (threadIdx.x < D) {
    float a = red[0][threadIdx.x];
    for (int j = 1; j < RPP; ++j) a = ABSMAX ? fmaxf(a, red[j][threadIdx.x]) : a + red[j][threadIdx.x];
    part[(bh * gridDim.x + ch) * D + threadIdx.x] = a;
  }
}

// Fixed-order fold of one statistic's slabs part[bh][chunk][d] by 256 threads (PARTS =
// 256 / D threads per channel, each folding a contiguous part of the chunks with eight
// independent partial results, then combined in a fixed order).  Returns the channel's
// total to the threads with threadIdx.x < D (d = threadIdx.x).  red: [256] floats of LDS.
template <int D, bool ABSMAX>
__device__ __forceinline__ float colfold(const float* __restrict__ part, int nch, int64_t bh, float* red) {
  constexpr int PARTS = 256 / D;
  const int d = threadIdx.x % D, p = threadIdx.x / D;
  const int c0 = p * nch / PARTS, c1 = (p + 1) * nch / PARTS;
  const float* src = part + (bh * nch) * D + d;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  int c = c0;
  for (; c + 8 <= c1; c += 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = src[(int64_t)(c + i) * D];
      acc[i] = ABSMAX ? fmaxf(acc[i], v) : acc[i] + v;
    }
  }
  for (; c < c1; ++c) {
    const float v = src[(int64_t)c * D];
    acc[0] = ABSMAX ? fmaxf(acc[0], v) : acc[0] + v;
  }
#pragma unroll
  for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) acc[i] = ABSMAX ? fmaxf(acc[i], acc[i + w]) : acc[i] + acc[i + w];
  red[p * D + d] = acc[0];
  __syncthreads();
  float a = 0.0f;
  if (p == 0) {
    a = red[d];
#pragma unroll
    for (int j = 1; j < PARTS; ++j) a = ABSMAX ? fmaxf(a, red[j * D + d]) : a + red[j * D + d];
  }
  __syncthreads();
  return a;
}

// Fold of the per-chunk slabs of one statistic (grid B*H): SUM -> out = sum / S (the key
// mean), ABSMAX -> out = max(amax, 1e-12) / 448 (the per-channel V scale).
template <int D, bool ABSMAX>
__global__ __launch_bounds__(256) void attn_colfold_kernel(const float* __restrict__ part, int nch, int64_t S,
                                                           float* __restrict__ out) {
  __shared__ float red[256];
  const int64_t bh = blockIdx.x;
  const float a = colfold<D, ABSMAX>(part, nch, bh, red);
  if (threadIdx.x < D) out[bh * D + threadIdx.x] = ABSMAX ? e4m3_scale(a) : __fdiv_rn(a, (float)S);
}

// V quantizer of one (128-key tile blk, b*H + h), transposed store: the block quantizes a
// 128-key x D tile with the per-channel scales sv and writes it transposed through LDS so
// that every v8t row segment is a full 128 bytes.  Thread t handles d-chunk (t % CPR) of
// the 4 consecutive keys 4 * (t / CPR + KQP * p) + 0..3.
template <int D>
struct QuantVLds {
  static constexpr int STRIDE = 128 + 4;  // LDS row stride of the transposed tile
  uint8_t tile[D * STRIDE];
  float s_sv[D];
  float s_r[D];
};

template <int DT, int D, bool VEC>
__device__ __forceinline__ void quant_v_tile(const void* __restrict__ src, const Strides4& st, int64_t H, int64_t S,
                                             int64_t Sp, const float* __restrict__ sv, uint8_t* __restrict__ v8t,
                                             int64_t blk, int64_t bh, QuantVLds<D>& L) {
  constexpr int CPR = D / 8;
  constexpr int KQP = 256 / CPR;  // key quads per pass
  constexpr int NP = 32 / KQP;    // passes over the 32 key quads of the tile
  constexpr int LDS_STRIDE = QuantVLds<D>::STRIDE;
  uint8_t* const tile = L.tile;
  float* const s_sv = L.s_sv;
  float* const s_r = L.s_r;
  const int64_t b = bh / H, h = bh % H;
  if (threadIdx.x < D) {
    const float s = sv[bh * D + threadIdx.x];
    s_sv[threadIdx.x] = s;
    s_r[threadIdx.x] = __fdiv_rn(1.0f, s);
  }
  __syncthreads();
  const void* base = static_cast<const char*>(src) + (b * st.b + h * st.h) * (int64_t)sizeof(typename Elem<DT>::T);
  const int cc = threadIdx.x % CPR;
  float scl[8], rcp[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    scl[i] = s_sv[cc * 8 + i];
    rcp[i] = s_r[cc * 8 + i];
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int kq = threadIdx.x / CPR + KQP * p;
    uint32_t col[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // col[i]: 4 key bytes of channel cc*8+i
    uint4 raw[VEC ? 4 : 1];
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t s = blk * 128 + kq * 4 + j;
        raw[j] = s < S ? raw8<DT>(base, st, s, cc * 8) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t s = blk * 128 + kq * 4 + j;
      float f[8];
      if (s < S) {
        if constexpr (VEC)
          cvt8<DT>(raw[j], f);
        else
          load8<DT, VEC>(base, st, s, cc * 8, f);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const uint32_t two = cvt2_e4m3(clamp448(div_by_scale(f[i], scl[i], rcp[i])),
                                       clamp448(div_by_scale(f[i + 1], scl[i + 1], rcp[i + 1])));
        col[i] |= (two & 0xffu) << (8 * j);
        col[i + 1] |= (two >> 8) << (8 * j);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint32_t*>(&tile[(cc * 8 + i) * LDS_STRIDE + kq * 4]) = col[i];
  }
  __syncthreads();
  // D rows x 128 bytes, 16 bytes per thread-step
  constexpr int CHUNKS = D * 8;
  for (int x = threadIdx.x; x < CHUNKS; x += 256) {
    const int d = x >> 3, kc = x & 7;
    const uint32_t* src4 = reinterpret_cast<const uint32_t*>(&tile[d * LDS_STRIDE + kc * 16]);
    uint4 o = make_uint4(src4[0], src4[1], src4[2], src4[3]);
    *reinterpret_cast<uint4*>(v8t + (bh * D + d) * Sp + blk * 128 + kc * 16) = o;
  }
}

// One block per (128-key tile, b*H + h).
template <int DT, int D, bool VEC>
__global__ __launch_bounds__(256) void attn_quant_v_kernel(const void* __restrict__ src, Strides4 st, int64_t H,
                                                           int64_t S, int64_t Sp, const float* __restrict__ sv,
                                                           uint8_t* __restrict__ v8t) {
  __shared__ QuantVLds<D> L;
  quant_v_tile<DT, D, VEC>(src, st, H, S, Sp, sv, v8t, blockIdx.x, blockIdx.y, L);
}

// ---------------------------------------------------------------------------------------
// K and V of one attention together (kernels/fp8_attention.py:338-369): one pass over both
// for the statistics that need the whole sequence (the key mean, the per-channel V amax),
// one fold of both, then one launch that quantizes a 128-key tile of K and of V per block.
// The second read of K and V follows the first closely, so it is mostly served by the
// MALL; in the fused QKV layout ([B, S, 2, H, D]) the two reads of a key's K and V rows
// are adjacent.
// ---------------------------------------------------------------------------------------

// Partial column statistics over a chunk of keys: part[0][bh][chunk][d] = sum of k,
// part[1][bh][chunk][d] = max |v| (grid (B*H, nch): heads fastest, so the blocks that run
// together read the same keys' rows, which in a [B, S, (2,) H, D] layout are adjacent).
template <int DT, int D, bool VECK, bool VECV>
__global__ __launch_bounds__(256) void attn_kv_colreduce_kernel(const void* __restrict__ k, Strides4 stk,
                                                                const void* __restrict__ v, Strides4 stv, int64_t H,
                                                                int64_t S, int64_t rows_per_chunk,
                                                                float* __restrict__ part) {
  constexpr int CPR = D / 8;
  constexpr int RPP = 256 / CPR;
  __shared__ float red[2][RPP][D + 1];
  const int64_t ch = blockIdx.y, nch = gridDim.y;
  const int64_t bh = blockIdx.x, BH = gridDim.x;
  const int64_t b = bh / H, h = bh % H;
  constexpr int64_t ES = sizeof(typename Elem<DT>::T);
  const void* kb = static_cast<const char*>(k) + (b * stk.b + h * stk.h) * ES;
  const void* vb = static_cast<const char*>(v) + (b * stv.b + h * stv.h) * ES;
  const int cc = threadIdx.x % CPR;
  const int rl = threadIdx.x / CPR;
  const int64_t r0 = ch * rows_per_chunk;
  const int64_t r1 = min(S, r0 + rows_per_chunk);
  float ks[8], va[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ks[i] = va[i] = 0.0f;
  int64_t s = r0 + rl;
  if constexpr (VECK && VECV) {
    // 4 rows of K and of V in flight together; rows are folded in the same order as one
    // at a time
    constexpr int U = 4;
    for (; s + (U - 1) * RPP < r1; s += U * RPP) {
      uint4 rk[U], rv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        rk[u] = raw8<DT>(kb, stk, s + u * RPP, cc * 8);
        rv[u] = raw8<DT>(vb, stv, s + u * RPP, cc * 8);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float fk[8], fv[8];
        cvt8<DT>(rk[u], fk);
        cvt8<DT>(rv[u], fv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ks[i] += fk[i];
          va[i] = fmaxf(va[i], fabsf(fv[i]));
        }
      }
    }
  }
  for (; s < r1; s += RPP) {
    float fk[8], fv[8];
    load8<DT, VECK>(kb, stk, s, cc * 8, fk);
    load8<DT, VECV>(vb, stv, s, cc * 8, fv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ks[i] += fk[i];
      va[i] = fmaxf(va[i], fabsf(fv[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    red[0][rl][cc * 8 + i] = ks[i];
    red[1][rl][cc * 8 + i] = va[i];
  }
  __syncthreads();
  if (threadIdx.x < 2 * D) {
    const int t = threadIdx.x / D, d = threadIdx.x % D;
    float a = red[t][0][d];
    for (int j = 1; j < RPP; ++j) a = t ? fmaxf(a, red[t][j][d]) : a + red[t][j][d];
    part[((t * BH + bh) * nch + ch) * D + d] = a;
  }
}

// Both folds (grid B*H): mean[bh][d] = sum / S, sv[bh][d] = max(amax, 1e-12) / 448.
template <int D>
__global__ __launch_bounds__(256) void attn_kv_fold_kernel(const float* __restrict__ part, int nch, int64_t S,
                                                           float* __restrict__ mean, float* __restrict__ sv) {
  __shared__ float red[256];
  const int64_t bh = blockIdx.x, BH = gridDim.x;
  const float sum = colfold<D, false>(part, nch, bh, red);
  const float amax = colfold<D, true>(part + BH * nch * D, nch, bh, red);
  if (threadIdx.x < D) {
    mean[bh * D + threadIdx.x] = __fdiv_rn(sum, (float)S);
    sv[bh * D + threadIdx.x] = e4m3_scale(amax);
  }
}

// K tile and V tile of the same 128 keys (grid (B*H, Skp/128)).
template <int DT, int D, bool VECK, bool VECV>
__global__ __launch_bounds__(256) void attn_quant_kv_kernel(const void* __restrict__ k, Strides4 stk,
                                                            const void* __restrict__ v, Strides4 stv, int64_t H,
                                                            int64_t S, int64_t Sp, const float* __restrict__ mean,
                                                            const float* __restrict__ sv, uint8_t* __restrict__ k8,
                                                            float* __restrict__ sk, uint8_t* __restrict__ v8t) {
  __shared__ float red[4];
  __shared__ QuantVLds<D> L;
  // heads fastest: blocks that run together read the same keys' rows
  const int64_t bh = blockIdx.x, blk = blockIdx.y, nb = gridDim.y;
  quant_qk_tile<DT, D, true, VECK>(k, stk, H, S, Sp, 0.0f, mean, k8, sk, blk, bh, nb, red);
  quant_v_tile<DT, D, VECV>(v, stv, H, S, Sp, sv, v8t, blk, bh, L);
}

// Fold of the K/V column statistics that the QKV projection's epilogue emits
// (mxf8_gemm_rowwise_kv_stats: part[stat][p][c], stat 0 key sums, 1 value |max|, over the
// 128-row blocks p that lie inside one batch item, c = h D + d).  One workgroup per (b, h)
// and statistic (blockIdx.y: 0 the key mean, 1 the V scales; only the V scales without
// key_stats).  The blocks of item b are p in [b S / 128, ((b + 1) S - 1) / 128]; the first
// and the last may hold rows of another item or rows past the end, and for those the item's
// rows are read from k / v themselves.  Thread t folds channel d = t % D from phase t / D
// (P = 1024 / D phases): every P-th row of such a block and every P-th clean block (24 loads
// in flight: one round for a 480p item), in row and block order; the phases are then
// combined in order.  mean = sum / S, sv = max(amax, 1e-12) / 448 (|max| skips NaN).
template <int DT, int D>
__global__ __launch_bounds__(1024) void gemm_kv_stats_fold_kernel(const float* __restrict__ part, int64_t nb,
                                                                  const void* __restrict__ k, Strides4 stk,
                                                                  const void* __restrict__ v, Strides4 stv,
                                                                  int64_t H, int64_t S, int key_stats,
                                                                  float* __restrict__ mean, float* __restrict__ sv) {
  constexpr int P = 1024 / D, U = 24, R = 128 / P;
  constexpr int64_t ES = sizeof(typename Elem<DT>::T);
  __shared__ float red[P][D];
  const int64_t bh = blockIdx.x, b = bh / H, h = bh % H, C = H * D;
  const bool vstat = blockIdx.y != 0 || !key_stats;  // without key statistics: one y index, the V scales
  const int d = threadIdx.x % D, ph = threadIdx.x / D;
  const int64_t r0 = b * S, p_lo = r0 / 128, p_hi = (r0 + S - 1) / 128;
  const float* const src = part + (vstat ? nb * C : 0) + h * D + d;
  const Strides4& st = vstat ? stv : stk;
  const typename Elem<DT>::T* const row0 = reinterpret_cast<const typename Elem<DT>::T*>(
      static_cast<const char*>(vstat ? v : k) + (b * st.b + h * st.h + d * st.d) * ES);
  float a = 0.0f;
  auto fold = [&](float x) { a = vstat ? fmaxf(a, fabsf(x)) : a + x; };
  // rows [s0, s1) of item b (s1 - s0 <= 128), every P-th from this phase: all loads issued
  // first (clamped indices), then folded in row order
  auto rows = [&](int64_t s0, int64_t s1) {
    float x[R];
#pragma unroll
    for (int u = 0; u < R; ++u) x[u] = Elem<DT>::to_f32(row0[min(s0 + ph + u * P, s1 - 1) * st.s]);
#pragma unroll
    for (int u = 0; u < R; ++u)
      if (s0 + ph + u * P < s1) fold(x[u]);
  };
  auto clean = [&](int64_t p) { return p * 128 >= r0 && p * 128 + 128 <= r0 + S; };
  int64_t pf = p_lo, pl = p_hi;
  if (!clean(p_lo)) {
    rows(0, min(p_lo * 128 + 128, r0 + S) - r0);
    ++pf;
  }
  const bool tail = pl >= pf && !clean(pl);
  if (tail) --pl;
  for (int64_t p0 = pf + ph; p0 <= pl; p0 += U * P) {
    float x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = src[min(p0 + u * P, pl) * C];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (p0 + u * P <= pl) {
        a = vstat ? fmaxf(a, x[u]) : a + x[u];
      }
  }
  if (tail) rows(p_hi * 128 - r0, S);
  red[ph][d] = a;
  __syncthreads();
  if (ph == 0) {
#pragma unroll
    for (int j = 1; j < P; ++j) a = vstat ? fmaxf(a, red[j][d]) : a + red[j][d];
    if (vstat)
      sv[bh * D + d] = e4m3_scale(a);
    else
      mean[bh * D + d] = __fdiv_rn(a, (float)S);
  }
}

static bool attn_vec_ok(const void* p, int dtype, const Strides4& st) {
  const int64_t es = dtype == MXF8_F32 ? 4 : 2;
  return st.d == 1 && ((uintptr_t)p % 16 == 0) && ((st.b * es) % 16 == 0) && ((st.h * es) % 16 == 0) &&
         ((st.s * es) % 16 == 0);
}

static int attn_common_checks(const char* what, const void* src, int dtype, int64_t B, int64_t H, int64_t S,
                              int64_t D) {
  if (!src) return set_error(MXF8_EINVAL, "%s: null input", what);
  if (dtype != MXF8_BF16 && dtype != MXF8_F16)
    return set_error(MXF8_EINVAL, "%s: dtype must be bf16 or fp16", what);
  if (D != 64 && D != 128) return set_error(MXF8_EINVAL, "%s: D must be 64 or 128 (got %lld)", what, (long long)D);
  if (B <= 0 || H <= 0 || S <= 0) return set_error(MXF8_EINVAL, "%s: empty shape", what);
  if (B * H > 65535) return set_error(MXF8_EINVAL, "%s: B*H must be <= 65535", what);
  return MXF8_OK;
}

// Number of row chunks for the column reductions: enough blocks to fill the chip.
static int colreduce_chunks(int64_t BH, int64_t S) {
  int64_t nch = cdiv(2048, BH);
  nch = nch < 1 ? 1 : nch;
  nch = nch > 64 ? 64 : nch;
  const int64_t max_by_rows = cdiv(S, 64);
  return (int)(nch < max_by_rows ? nch : max_by_rows);
}

}  // namespace mxf8

using namespace mxf8;

extern "C" int mxf8_quant_rows(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* x8,
                               float* scale, hipStream_t stream) {
  if (M < 0 || K < 0) return set_error(MXF8_EINVAL, "quant_rows: negative shape");
  if (M == 0) return MXF8_OK;
  if (!scale) return set_error(MXF8_EINVAL, "quant_rows: null scale");
  if (K == 0) {
    fill_f32_kernel<<<dim3((unsigned)cdiv(M, 256)), dim3(256), 0, stream>>>(scale, M, kScaleFloor / kE4m3Max);
    return check_launch("quant_rows(fill)");
  }
  if (!x || !x8) return set_error(MXF8_EINVAL, "quant_rows: null pointer");
  if (ldx < K) return set_error(MXF8_EINVAL, "quant_rows: ldx < K");
  switch (dtype) {
    case MXF8_BF16: return quant_rows_dispatch<MXF8_BF16>(x, M, K, ldx, x8, scale, stream);
    case MXF8_F16: return quant_rows_dispatch<MXF8_F16>(x, M, K, ldx, x8, scale, stream);
    case MXF8_F32: return quant_rows_dispatch<MXF8_F32>(x, M, K, ldx, x8, scale, stream);
    default: return set_error(MXF8_EINVAL, "quant_rows: unknown dtype %d", dtype);
  }
}

extern "C" int mxf8_adaln_quant_rows(const void* x, int64_t M, int64_t C, int64_t ldx, int64_t S, const void* shift,
                                     const void* scale, int64_t ldm, float eps, int eager, uint8_t* x8, float* sa,
                                     void* y, hipStream_t stream) {
  if (M < 0 || C <= 0 || S <= 0) return set_error(MXF8_EINVAL, "adaln_quant_rows: bad shape");
  if (M == 0) return MXF8_OK;
  if (!x || !shift || !scale || !x8 || !sa) return set_error(MXF8_EINVAL, "adaln_quant_rows: null pointer");
  if (C % 8 || ldx % 8 || ldm % 8 || ldx < C || ldm < C)
    return set_error(MXF8_EINVAL, "adaln_quant_rows: C, ldx, ldm must be multiples of 8 with ldx, ldm >= C");
  if (((uintptr_t)x | (uintptr_t)shift | (uintptr_t)scale | (uintptr_t)x8 | (uintptr_t)y) % 16)
    return set_error(MXF8_EINVAL, "adaln_quant_rows: operands must be 16-byte aligned");
  const int64_t per_lane = cdiv(C / 8, 64);
  if (per_lane > 16) return set_error(MXF8_EINVAL, "adaln_quant_rows: C=%lld exceeds 8192", (long long)C);
  if (cdiv(M, 4) > 0x7fffffff) return set_error(MXF8_EINVAL, "adaln_quant_rows: M too large");
  if (!(eps >= 0.0f)) return set_error(MXF8_EINVAL, "adaln_quant_rows: eps must be >= 0");
  const int nc = per_lane <= 1 ? 1 : per_lane <= 2 ? 2 : per_lane <= 4 ? 4 : per_lane <= 6 ? 6 : per_lane <= 8 ? 8
                 : per_lane <= 12 ? 12 : 16;
  const uint16_t* x16 = static_cast<const uint16_t*>(x);
  const uint16_t* sh = static_cast<const uint16_t*>(shift);
  const uint16_t* sc = static_cast<const uint16_t*>(scale);
  uint16_t* y16 = static_cast<uint16_t*>(y);
  if (eager)
    adaln_dispatch<true>(nc, x16, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y16, stream);
  else
    adaln_dispatch<false>(nc, x16, M, C, ldx, S, sh, sc, ldm, eps, x8, sa, y16, stream);
  return check_launch("adaln_quant_rows");
}

extern "C" int64_t mxf8_attn_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D) {
  (void)Sq;
  if (B <= 0 || H <= 0 || Sk <= 0 || D <= 0) return 0;
  return (int64_t)colreduce_chunks(B * H, Sk) * B * H * D * (int64_t)sizeof(float);
}

template <int DT, int D, bool IS_K>
static void launch_qk(const void* src, const Strides4& st, bool vec, int64_t H, int64_t S, int64_t BH, float c,
                      const float* mean, uint8_t* out8, float* sc, hipStream_t stream) {
  const int64_t nb = cdiv(S, 128);
  dim3 grid((unsigned)nb, (unsigned)BH);
  if (vec)
    attn_quant_qk_kernel<DT, D, IS_K, true><<<grid, 256, 0, stream>>>(src, st, H, S, nb * 128, c, mean, out8, sc);
  else
    attn_quant_qk_kernel<DT, D, IS_K, false><<<grid, 256, 0, stream>>>(src, st, H, S, nb * 128, c, mean, out8, sc);
}

template <bool IS_K>
static int quant_qk(const char* what, const void* src, int dtype, const int64_t strides[4], const float* mean,
                    int64_t B, int64_t H, int64_t S, int64_t D, float c, uint8_t* out8, float* sc,
                    hipStream_t stream) {
  int rc = attn_common_checks(what, src, dtype, B, H, S, D);
  if (rc) return rc;
  if (!strides || !out8 || !sc || (IS_K && !mean)) return set_error(MXF8_EINVAL, "%s: null pointer", what);
  if (cdiv(S, 128) > 0x7fffffff) return set_error(MXF8_EINVAL, "%s: S too large", what);
  const Strides4 st{strides[0], strides[1], strides[2], strides[3]};
  const bool vec = attn_vec_ok(src, dtype, st);
  const int64_t BH = B * H;
  if (dtype == MXF8_BF16) {
    if (D == 128) launch_qk<MXF8_BF16, 128, IS_K>(src, st, vec, H, S, BH, c, mean, out8, sc, stream);
    else launch_qk<MXF8_BF16, 64, IS_K>(src, st, vec, H, S, BH, c, mean, out8, sc, stream);
  } else {
    if (D == 128) launch_qk<MXF8_F16, 128, IS_K>(src, st, vec, H, S, BH, c, mean, out8, sc, stream);
    else launch_qk<MXF8_F16, 64, IS_K>(src, st, vec, H, S, BH, c, mean, out8, sc, stream);
  }
  return check_launch(what);
}

extern "C" int mxf8_attn_quant_q(const void* q, int dtype, const int64_t strides[4], int64_t B, int64_t H,
                                 int64_t S, int64_t D, float c, uint8_t* q8, float* sq, hipStream_t stream) {
  return quant_qk<false>("attn_quant_q", q, dtype, strides, nullptr, B, H, S, D, c, q8, sq, stream);
}

extern "C" int mxf8_attn_quant_k(const void* k, int dtype, const int64_t strides[4], const float* mean,
                                 int64_t B, int64_t H, int64_t S, int64_t D, uint8_t* k8, float* sk,
                                 hipStream_t stream) {
  return quant_qk<true>("attn_quant_k", k, dtype, strides, mean, B, H, S, D, 0.0f, k8, sk, stream);
}

template <int DT, int D, bool ABSMAX>
static void launch_colreduce(const void* src, const Strides4& st, bool vec, int64_t H, int64_t S, int64_t BH,
                             int nch, float* part, hipStream_t stream) {
  const int64_t rpc = cdiv(S, nch);
  dim3 grid((unsigned)nch, (unsigned)BH);
  if (vec)
    attn_colreduce_kernel<DT, D, ABSMAX, true><<<grid, 256, 0, stream>>>(src, st, H, S, rpc, part);
  else
    attn_colreduce_kernel<DT, D, ABSMAX, false><<<grid, 256, 0, stream>>>(src, st, H, S, rpc, part);
}

template <bool ABSMAX>
static void colreduce(const void* src, int dtype, const Strides4& st, bool vec, int64_t H, int64_t S, int64_t D,
                      int64_t BH, int nch, float* part, hipStream_t stream) {
  if (dtype == MXF8_BF16) {
    if (D == 128) launch_colreduce<MXF8_BF16, 128, ABSMAX>(src, st, vec, H, S, BH, nch, part, stream);
    else launch_colreduce<MXF8_BF16, 64, ABSMAX>(src, st, vec, H, S, BH, nch, part, stream);
  } else {
    if (D == 128) launch_colreduce<MXF8_F16, 128, ABSMAX>(src, st, vec, H, S, BH, nch, part, stream);
    else launch_colreduce<MXF8_F16, 64, ABSMAX>(src, st, vec, H, S, BH, nch, part, stream);
  }
}

extern "C" int mxf8_attn_kmean(const void* k, int dtype, const int64_t strides[4], int64_t B, int64_t H,
                               int64_t S, int64_t D, float* mean, void* workspace, hipStream_t stream) {
  int rc = attn_common_checks("attn_kmean", k, dtype, B, H, S, D);
  if (rc) return rc;
  if (!strides || !mean || !workspace) return set_error(MXF8_EINVAL, "attn_kmean: null pointer");
  const Strides4 st{strides[0], strides[1], strides[2], strides[3]};
  const int64_t BH = B * H;
  const int nch = colreduce_chunks(BH, S);
  float* part = static_cast<float*>(workspace);
  colreduce<false>(k, dtype, st, attn_vec_ok(k, dtype, st), H, S, D, BH, nch, part, stream);
  rc = check_launch("attn_kmean(partial)");
  if (rc) return rc;
  if (D == 128)
    attn_colfold_kernel<128, false><<<dim3((unsigned)BH), dim3(256), 0, stream>>>(part, nch, S, mean);
  else
    attn_colfold_kernel<64, false><<<dim3((unsigned)BH), dim3(256), 0, stream>>>(part, nch, S, mean);
  return check_launch("attn_kmean(fold)");
}

template <int DT, int D>
static void launch_quant_v(const void* v, const Strides4& st, bool vec, int64_t H, int64_t S, int64_t BH,
                           const float* sv, uint8_t* v8t, hipStream_t stream) {
  const int64_t nb = cdiv(S, 128);
  dim3 grid((unsigned)nb, (unsigned)BH);
  if (vec)
    attn_quant_v_kernel<DT, D, true><<<grid, 256, 0, stream>>>(v, st, H, S, nb * 128, sv, v8t);
  else
    attn_quant_v_kernel<DT, D, false><<<grid, 256, 0, stream>>>(v, st, H, S, nb * 128, sv, v8t);
}

extern "C" int mxf8_attn_quant_v(const void* v, int dtype, const int64_t strides[4], int64_t B, int64_t H,
                                 int64_t S, int64_t D, uint8_t* v8t, float* sv, void* workspace,
                                 hipStream_t stream) {
  int rc = attn_common_checks("attn_quant_v", v, dtype, B, H, S, D);
  if (rc) return rc;
  if (!strides || !v8t || !sv || !workspace) return set_error(MXF8_EINVAL, "attn_quant_v: null pointer");
  const Strides4 st{strides[0], strides[1], strides[2], strides[3]};
  const bool vec = attn_vec_ok(v, dtype, st);
  const int64_t BH = B * H;
  const int nch = colreduce_chunks(BH, S);
  float* part = static_cast<float*>(workspace);
  colreduce<true>(v, dtype, st, vec, H, S, D, BH, nch, part, stream);
  rc = check_launch("attn_quant_v(absmax)");
  if (rc) return rc;
  if (D == 128)
    attn_colfold_kernel<128, true><<<dim3((unsigned)BH), dim3(256), 0, stream>>>(part, nch, S, sv);
  else
    attn_colfold_kernel<64, true><<<dim3((unsigned)BH), dim3(256), 0, stream>>>(part, nch, S, sv);
  rc = check_launch("attn_quant_v(scale)");
  if (rc) return rc;
  if (dtype == MXF8_BF16) {
    if (D == 128) launch_quant_v<MXF8_BF16, 128>(v, st, vec, H, S, BH, sv, v8t, stream);
    else launch_quant_v<MXF8_BF16, 64>(v, st, vec, H, S, BH, sv, v8t, stream);
  } else {
    if (D == 128) launch_quant_v<MXF8_F16, 128>(v, st, vec, H, S, BH, sv, v8t, stream);
    else launch_quant_v<MXF8_F16, 64>(v, st, vec, H, S, BH, sv, v8t, stream);
  }
  return check_launch("attn_quant_v");
}

extern "C" int64_t mxf8_attn_kv_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D) {
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0) return 0;
  const int64_t BH = B * H;
  // partial slabs of both statistics, then the key mean
  return (2 * (int64_t)colreduce_chunks(BH, S) + 1) * BH * D * (int64_t)sizeof(float);
}

template <int DT, int D>
static void launch_kv(const void* k, const Strides4& stk, bool veck, const void* v, const Strides4& stv, bool vecv,
                      int64_t H, int64_t S, int64_t BH, int nch, float* part, float* mean, float* sv, uint8_t* k8,
                      float* sk, uint8_t* v8t, hipStream_t stream) {
  const int64_t rpc = cdiv(S, nch);
  const dim3 rgrid((unsigned)BH, (unsigned)nch);
  const int64_t nb = cdiv(S, 128);
  const dim3 qgrid((unsigned)BH, (unsigned)nb);
#define MXF8_KV_CASE(VK, VV)                                                                                     \
  if (veck == VK && vecv == VV) {                                                                                \
    attn_kv_colreduce_kernel<DT, D, VK, VV><<<rgrid, 256, 0, stream>>>(k, stk, v, stv, H, S, rpc, part);         \
    attn_kv_fold_kernel<D><<<dim3((unsigned)BH), 256, 0, stream>>>(part, nch, S, mean, sv);                       \
    attn_quant_kv_kernel<DT, D, VK, VV><<<qgrid, 256, 0, stream>>>(k, stk, v, stv, H, S, nb * 128, mean, sv, k8, \
                                                                    sk, v8t);                                    \
    return;                                                                                                      \
  }
  MXF8_KV_CASE(true, true)
  MXF8_KV_CASE(true, false)
  MXF8_KV_CASE(false, true)
  MXF8_KV_CASE(false, false)
#undef MXF8_KV_CASE
}

// The quantizing pass of the K/V pair alone (the key mean and V scales given).
template <int DT, int D>
static void launch_quant_kv_only(const void* k, const Strides4& stk, bool veck, const void* v, const Strides4& stv,
                                 bool vecv, int64_t H, int64_t S, int64_t BH, const float* mean, const float* sv,
                                 uint8_t* k8, float* sk, uint8_t* v8t, hipStream_t stream) {
  const int64_t nb = cdiv(S, 128);
  const dim3 qgrid((unsigned)BH, (unsigned)nb);
#define MXF8_KVQ_CASE(VK, VV)                                                                                    \
  if (veck == VK && vecv == VV) {                                                                                \
    attn_quant_kv_kernel<DT, D, VK, VV><<<qgrid, 256, 0, stream>>>(k, stk, v, stv, H, S, nb * 128, mean, sv, k8, \
                                                                    sk, v8t);                                    \
    return;                                                                                                      \
  }
  MXF8_KVQ_CASE(true, true)
  MXF8_KVQ_CASE(true, false)
  MXF8_KVQ_CASE(false, true)
  MXF8_KVQ_CASE(false, false)
#undef MXF8_KVQ_CASE
}

// K and V quantized together: the key mean, the K quantizer, the per-channel V scale and
// the transposed V quantizer (kernels/fp8_attention.py:338-369) in three launches.
static int attn_quant_kv_impl(const char* what, const void* k, const int64_t k_strides[4], const void* v,
                              const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                              uint8_t* k8, float* sk, uint8_t* v8t, float* sv, float* mean, float* part, int nch,
                              hipStream_t stream) {
  const Strides4 stk{k_strides[0], k_strides[1], k_strides[2], k_strides[3]};
  const Strides4 stv{v_strides[0], v_strides[1], v_strides[2], v_strides[3]};
  const bool veck = attn_vec_ok(k, dtype, stk), vecv = attn_vec_ok(v, dtype, stv);
  const int64_t BH = B * H;
  if (dtype == MXF8_BF16) {
    if (D == 128) launch_kv<MXF8_BF16, 128>(k, stk, veck, v, stv, vecv, H, S, BH, nch, part, mean, sv, k8, sk, v8t, stream);
    else launch_kv<MXF8_BF16, 64>(k, stk, veck, v, stv, vecv, H, S, BH, nch, part, mean, sv, k8, sk, v8t, stream);
  } else {
    if (D == 128) launch_kv<MXF8_F16, 128>(k, stk, veck, v, stv, vecv, H, S, BH, nch, part, mean, sv, k8, sk, v8t, stream);
    else launch_kv<MXF8_F16, 64>(k, stk, veck, v, stv, vecv, H, S, BH, nch, part, mean, sv, k8, sk, v8t, stream);
  }
  return check_launch(what);
}

static int attn_quant_kv_checks(const char* what, const void* k, const int64_t k_strides[4], const void* v,
                                const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                const uint8_t* k8, const float* sk, const uint8_t* v8t, const float* sv) {
  int rc = attn_common_checks(what, k, dtype, B, H, S, D);
  if (rc) return rc;
  if (!v || !k_strides || !v_strides || !k8 || !sk || !v8t || !sv)
    return set_error(MXF8_EINVAL, "%s: null pointer", what);
  // the quantizer's grid has one y index per 128-key tile
  if (cdiv(S, 128) > 65535) return set_error(MXF8_EINVAL, "%s: S must be <= %d", what, 65535 * 128);
  return MXF8_OK;
}

extern "C" int mxf8_attn_quant_kv(const void* k, const int64_t k_strides[4], const void* v,
                                  const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                  uint8_t* k8, float* sk, uint8_t* v8t, float* sv, float* mean, void* workspace,
                                  hipStream_t stream) {
  const char* what = "attn_quant_kv";
  int rc = attn_quant_kv_checks(what, k, k_strides, v, v_strides, dtype, B, H, S, D, k8, sk, v8t, sv);
  if (rc) return rc;
  if (!workspace) return set_error(MXF8_EINVAL, "%s: null workspace", what);
  const int64_t BH = B * H;
  const int nch = colreduce_chunks(BH, S);
  float* part = static_cast<float*>(workspace);
  float* mean_ws = part + 2 * (int64_t)nch * BH * D;
  return attn_quant_kv_impl(what, k, k_strides, v, v_strides, dtype, B, H, S, D, k8, sk, v8t, sv,
                            mean ? mean : mean_ws, part, nch, stream);
}

// K and V quantized from the column statistics of the QKV projection that produced them
// (mxf8_gemm_rowwise_kv_stats): one fold launch for the key mean and the V scales, then the
// quantizing pass -- K and V are read once.
extern "C" int mxf8_attn_quant_kv_gemm_stats(const void* k, const int64_t k_strides[4], const void* v,
                                             const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S,
                                             int64_t D, const float* part, int key_stats, uint8_t* k8, float* sk,
                                             uint8_t* v8t, float* sv, float* mean, hipStream_t stream) {
  const char* what = "attn_quant_kv_gemm_stats";
  int rc = attn_quant_kv_checks(what, k, k_strides, v, v_strides, dtype, B, H, S, D, k8, sk, v8t, sv);
  if (rc) return rc;
  if (!part || !mean) return set_error(MXF8_EINVAL, "%s: null statistics or mean", what);
  if (S < 128) return set_error(MXF8_EINVAL, "%s: S=%lld must be >= 128", what, (long long)S);
  if ((H * D) % 256) return set_error(MXF8_EINVAL, "%s: H*D must be a multiple of 256", what);
  if (B * S > (1 << 30)) return set_error(MXF8_EINVAL, "%s: B*S too large", what);
  const Strides4 stk{k_strides[0], k_strides[1], k_strides[2], k_strides[3]};
  const Strides4 stv{v_strides[0], v_strides[1], v_strides[2], v_strides[3]};
  const bool veck = attn_vec_ok(k, dtype, stk), vecv = attn_vec_ok(v, dtype, stv);
  const int64_t BH = B * H, nb = cdiv(B * S, 128);
  // grid y: the key mean (only when it comes from part) and the V scales
  const dim3 fgrid((unsigned)BH, key_stats ? 2u : 1u);
#define MXF8_FOLD(DT_, D_)                                                                                         \
  gemm_kv_stats_fold_kernel<DT_, D_><<<fgrid, 1024, 0, stream>>>(part, nb, k, stk, v, stv, H, S, key_stats, mean, \
                                                                  sv)
  if (dtype == MXF8_BF16) {
    if (D == 128) MXF8_FOLD(MXF8_BF16, 128); else MXF8_FOLD(MXF8_BF16, 64);
  } else {
    if (D == 128) MXF8_FOLD(MXF8_F16, 128); else MXF8_FOLD(MXF8_F16, 64);
  }
#undef MXF8_FOLD
  rc = check_launch("attn_quant_kv_gemm_stats(fold)");
  if (rc) return rc;
  if (dtype == MXF8_BF16) {
    if (D == 128) launch_quant_kv_only<MXF8_BF16, 128>(k, stk, veck, v, stv, vecv, H, S, BH, mean, sv, k8, sk, v8t, stream);
    else launch_quant_kv_only<MXF8_BF16, 64>(k, stk, veck, v, stv, vecv, H, S, BH, mean, sv, k8, sk, v8t, stream);
  } else {
    if (D == 128) launch_quant_kv_only<MXF8_F16, 128>(k, stk, veck, v, stv, vecv, H, S, BH, mean, sv, k8, sk, v8t, stream);
    else launch_quant_kv_only<MXF8_F16, 64>(k, stk, veck, v, stv, vecv, H, S, BH, mean, sv, k8, sk, v8t, stream);
  }
  return check_launch(what);
}

// ---------------------------------------------------------------------------------------
// No-allocation form of mxf8_attn_quant_kv for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
// Its workspace is a file-scope device array: each GPU the library runs on holds its own
// copy until the process ends.  Host code never uses the array's name as an address: the
// entry point's first call on a device (that device current) looks up the device's copy
// with hipGetSymbolAddress and keeps it.  Every call on one GPU shares that GPU's copy, so
// two calls must not overlap on one GPU: outside graph capture the entry point orders them
// itself (a call on another stream than the previous one first waits for that call's event),
// while calls captured into a graph are ordered only by how the graph's replays are issued.
// Nothing in the array needs clearing: every partial slab and the key mean are written before
// they are read.
// ---------------------------------------------------------------------------------------
// 4 MiB: enough for every B*H <= 1638 at D = 128 (<= 5461 at D = 64)
constexpr int64_t kNoAllocScratchBytes = (int64_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;
// Per device: an event recorded after the last call made outside graph capture, and that
// call's stream (created with the device's scratch lookup; guarded by g_scratch_mu).
struct NoAllocOrder {
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool used = false;
};
NoAllocOrder g_noalloc_order[kMaxDevices];

// This device's copy of `scratch` (looked up once per device, with the device current; the
// device's ordering event is created then too).  *dev_out: the current device.
int scratch_ptr(const char* what, void** out, int* dev_out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(MXF8_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(MXF8_EINVAL, "%s: device %d out of range", what, dev);
  void* p = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_dev[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return set_error(MXF8_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", what, hipGetErrorString(e));
      e = hipEventCreateWithFlags(&g_noalloc_order[dev].done, hipEventDisableTiming);
      if (e != hipSuccess)
        return set_error(MXF8_ELAUNCH, "%s: hipEventCreateWithFlags failed: %s", what, hipGetErrorString(e));
      g_scratch_dev[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  *dev_out = dev;
  return MXF8_OK;
}
}  // namespace

extern "C" int mxf8_attn_quant_kv_noalloc(const void* k, const int64_t k_strides[4], const void* v,
                                          const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S,
                                          int64_t D, uint8_t* k8, float* sk, uint8_t* v8t, float* sv, float* mean,
                                          hipStream_t stream) {
  const char* what = "attn_quant_kv_noalloc";
  int rc = attn_quant_kv_checks(what, k, k_strides, v, v_strides, dtype, B, H, S, D, k8, sk, v8t, sv);
  if (rc) return rc;
  const int64_t need = mxf8_attn_kv_workspace_bytes(B, H, S, D);
  if (need > kNoAllocScratchBytes)
    return set_error(MXF8_EINVAL,
                     "%s: B*H=%lld, S=%lld, D=%lld need %lld bytes of scratch, more than its %lld (use "
                     "mxf8_attn_quant_kv with a workspace)",
                     what, (long long)(B * H), (long long)S, (long long)D, (long long)need,
                     (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  int dev = 0;
  rc = scratch_ptr(what, &ws, &dev);
  if (rc) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) return set_error(MXF8_ELAUNCH, "%s: hipStreamIsCapturing failed: %s", what, hipGetErrorString(e));
  const bool ordered = cap == hipStreamCaptureStatusNone;
  const int64_t BH = B * H;
  const int nch = colreduce_chunks(BH, S);  // as mxf8_attn_quant_kv: the same sums, bit for bit
  float* part = static_cast<float*>(ws);
  float* mean_ws = part + 2 * (int64_t)nch * BH * D;
  // the wait, the launches and the record stay together, so that calls from several threads
  // are ordered as well
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  NoAllocOrder& ord = g_noalloc_order[dev];
  if (ordered && ord.used && ord.last != stream) {
    e = hipStreamWaitEvent(stream, ord.done, 0);
    if (e != hipSuccess) return set_error(MXF8_ELAUNCH, "%s: hipStreamWaitEvent failed: %s", what, hipGetErrorString(e));
  }
  rc = attn_quant_kv_impl(what, k, k_strides, v, v_strides, dtype, B, H, S, D, k8, sk, v8t, sv,
                          mean ? mean : mean_ws, part, nch, stream);
  if (rc) return rc;
  if (ordered) {
    e = hipEventRecord(ord.done, stream);
    if (e != hipSuccess) return set_error(MXF8_ELAUNCH, "%s: hipEventRecord failed: %s", what, hipGetErrorString(e));
    ord.last = stream;
    ord.used = true;
  }
  return MXF8_OK;
}
