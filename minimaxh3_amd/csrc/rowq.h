// Per-row pieces of the activation quantizers, for a bf16 row held by one wave: NC 16-byte
// chunks per lane, chunk c of lane l holding elements [(c * 64 + l) * 8, +8) (chunks past the
// row's end hold zeros).  Used by adaln_quant_rows_kernel.
#pragma once

#include "common.h"

namespace mxf8 {

// Loads row xr (nchunk = K / 8 chunks) into v; chunks past the end read as zeros.
template <int NC>
__device__ __forceinline__ void row_load_bf16(const uint16_t* __restrict__ xr, int64_t nchunk, int lane,
                                              uint4 (&v)[NC]) {
  const uint4* x4 = reinterpret_cast<const uint4*>(xr);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t idx = (int64_t)c * 64 + lane;
    v[c] = idx < nchunk ? x4[idx] : make_uint4(0, 0, 0, 0);
  }
}

// max |x| over this lane's elements of the row.
template <int NC>
__device__ __forceinline__ float row_absmax_bf16(const uint4 (&v)[NC]) {
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      amax = fmaxf(amax, fmaxf(fabsf(Elem<MXF8_BF16>::lo(w[i])), fabsf(Elem<MXF8_BF16>::hi(w[i]))));
  }
  return amax;
}

__device__ __forceinline__ float bf16_rne(float f) { return (float)(__bf16)f; }

// adaLN modulation of the row in place: y = LN(x) * (1 + scale) + shift with LayerNorm
// without affine (fp32 mean and biased variance, rstd = 1 / sqrt(var + eps)).  EAGER = false
// rounds y to bf16 once (the fused pointwise code of a compiled block); EAGER = true rounds
// after each of torch's eager bf16 ops (n, 1 + scale, product, sum).  shr / scr: the row's
// batch item's shift / scale as 16-byte chunks.  Returns max |y| over this lane's elements.
template <int NC, bool EAGER>
__device__ __forceinline__ float adaln_modulate_bf16(uint4 (&v)[NC], int64_t C, int64_t nchunk, int lane,
                                                     const uint4* __restrict__ shr, const uint4* __restrict__ scr,
                                                     float eps) {
  float sum = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) sum += Elem<MXF8_BF16>::lo(w[i]) + Elem<MXF8_BF16>::hi(w[i]);
  }
  const float mean = __fdiv_rn(wave_sum(sum), (float)C);
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t idx = (int64_t)c * 64 + lane;
    if (idx < nchunk) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d0 = Elem<MXF8_BF16>::lo(w[i]) - mean, d1 = Elem<MXF8_BF16>::hi(w[i]) - mean;
        ss = __builtin_fmaf(d0, d0, ss);
        ss = __builtin_fmaf(d1, d1, ss);
      }
    }
  }
  const float var = __fdiv_rn(wave_sum(ss), (float)C);
  const float rstd = __fdiv_rn(1.0f, __fsqrt_rn(var + eps));
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t idx = (int64_t)c * 64 + lane;
    if (idx < nchunk) {
      const uint4 sh = shr[idx], sc = scr[idx];
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
      const uint32_t hw[4] = {sh.x, sh.y, sh.z, sh.w}, cw[4] = {sc.x, sc.y, sc.z, sc.w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float yy[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float xf = h ? Elem<MXF8_BF16>::hi(w[i]) : Elem<MXF8_BF16>::lo(w[i]);
          const float shf = h ? Elem<MXF8_BF16>::hi(hw[i]) : Elem<MXF8_BF16>::lo(hw[i]);
          const float scf = h ? Elem<MXF8_BF16>::hi(cw[i]) : Elem<MXF8_BF16>::lo(cw[i]);
          const float n = (xf - mean) * rstd;
          if constexpr (EAGER)
            yy[h] = bf16_rne(bf16_rne(bf16_rne(n) * bf16_rne(1.0f + scf)) + shf);
          else
            yy[h] = bf16_rne(n * (1.0f + scf) + shf);
          amax = fmaxf(amax, fabsf(yy[h]));
        }
        o[i] = (__float_as_uint(yy[0]) >> 16) | (__float_as_uint(yy[1]) & 0xffff0000u);
      }
      v[c] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  return amax;
}

// e4m3 codes of the row at scale s (r = 1 / s correctly rounded) -> orow (K bytes).
template <int NC>
__device__ __forceinline__ void row_store_codes_bf16(const uint4 (&v)[NC], int64_t nchunk, int lane, float s, float r,
                                                     uint8_t* __restrict__ orow) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t idx = (int64_t)c * 64 + lane;
    if (idx < nchunk) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
      float f[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = clamp448(div_by_scale(Elem<MXF8_BF16>::lo(w[i]), s, r));
        f[2 * i + 1] = clamp448(div_by_scale(Elem<MXF8_BF16>::hi(w[i]), s, r));
      }
      *reinterpret_cast<uint2*>(orow + idx * 8) = make_uint2(cvt4_e4m3(f[0], f[1], f[2], f[3]),
                                                             cvt4_e4m3(f[4], f[5], f[6], f[7]));
    }
  }
}

}  // namespace mxf8
