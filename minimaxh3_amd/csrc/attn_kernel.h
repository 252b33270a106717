// FP8 flash-attention forward for gfx950 (non-causal; optional per-key mask / bias).
//
// Algorithm (kernels/fp8_attention.py:215-297, BLOCK_M = BLOCK_N = 128): per (b, h, Q tile
// I of 128 rows) the KV tiles are visited in the staggered order j = (j0 + i) % nk with
// j0 = I*nk/nq; scores are in the log2 domain S = (Q8 K8^T) * sq * sk; the row max m is
// lazy (it moves to the tile max only when that exceeds m + 8, or on the first valid
// tile); P is produced without exp2 as the e4m3 code rint(8 S + 56 - 8 m) (0 below 8);
// l += sum(P); O += P V; with repair_tau >= 0, exp2(S - m) - P is added for codes >= tau
// through bf16.  Output = O * sv / max(l, 1e-12).
//
// Mapping to CDNA4.  A workgroup (4 waves) owns one Q tile; wave w owns its 32 rows.  The
// kernel computes the TRANSPOSED score tile S^T = K Q^T with v_mfma_f32_32x32x64_f8f6f4:
// in the 32x32 accumulator layout lane l holds query column l%32, so every softmax row
// statistic is lane-local (plus one exchange with lane l^32).  The K rows of each 32-key
// subtile are fed to the MFMA in a permuted order chosen so that the accumulator
// registers, packed 4 per dword, ARE the B operand of the PV MFMA (O^T = V^T P^T) with
// V^T read as contiguous 32-byte runs of a v8t row: no cross-lane shuffles between the
// two products.  K and V^T tiles (and the mask / bias of the tile) are copied global ->
// LDS by the direct-to-LDS DMA, double-buffered.
#pragma once

#include "common.h"

namespace mxf8 {

__device__ __forceinline__ void attn_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Key (within a 128-key tile) of accumulator row R of score subtile t, and of register i
// of lane group g.  Subtile t covers keys 64(t/2) + 16(t%2) + {0..15, 32..47}.
__host__ __device__ constexpr int key_of_row(int t, int R) {
  return 64 * (t >> 1) + 16 * (t & 1) + 32 * ((R >> 2) & 1) + 4 * (R >> 3) + (R & 3);
}

template <int D>
struct AttnTile {
  static constexpr int KB = 128 * D;    // K tile bytes (128 keys x D)
  static constexpr int VB = D * 128;    // V^T tile bytes (D rows x 128 keys)
  static constexpr int AUXB = 2048;     // bias (1 KB slot) + mask (1 KB slot)
  static constexpr int CPRK = D / 16;   // 16-byte chunks per K row
  static constexpr int K_INSTR = KB / 1024 / 4;  // DMA instructions per wave
  static constexpr int V_INSTR = VB / 1024 / 4;
};

template <int D>
__device__ __forceinline__ v8i lds_read32(const uint8_t* tile, int row, int row_bytes, int cpr, int chunk0) {
  const int sw = row & (cpr - 1);
  const v4i lo = *reinterpret_cast<const v4i*>(tile + row * row_bytes + ((chunk0 ^ sw) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(tile + row * row_bytes + (((chunk0 + 1) ^ sw) << 4));
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// DMA one KV tile (keys [kv0, kv0 + 128)) of head bh into LDS buffers.
template <int D, bool HAS_MASK, bool HAS_BIAS>
__device__ __forceinline__ void attn_dma(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                         __amdgpu_buffer_rsrc_t brs, __amdgpu_buffer_rsrc_t mrs, uint8_t* sK,
                                         uint8_t* sV, uint8_t* sAux, uint32_t k_lane, uint32_t v_lane, int wave,
                                         int lane, int kv0, int Skp, int Sk, const float* bias_row,
                                         const uint8_t* mask_row) {
  typedef AttnTile<D> T;
  constexpr int RPI = 64 / T::CPRK;  // K rows per 1 KB instruction
#pragma unroll
  for (int j = 0; j < T::K_INSTR; ++j) {
    const int J = wave * T::K_INSTR + j;
    // LDS rows [RPI*J, RPI*J + RPI): accumulator row R of subtile t = R/32 loads key key_of_row.
    int ubase;
    if constexpr (D == 128) {
      const int t = J >> 2;
      ubase = 64 * (t >> 1) + 16 * (t & 1) + 4 * (J & 3);
    } else {
      const int t = J >> 1;
      ubase = 64 * (t >> 1) + 16 * (t & 1) + 8 * (J & 1);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, LDS_PTR(sK + J * 1024), 16, k_lane, (kv0 + ubase) * D, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < T::V_INSTR; ++j) {
    const int J = wave * T::V_INSTR + j;  // V^T rows [8J, 8J + 8)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, LDS_PTR(sV + J * 1024), 16, v_lane, 8 * J * Skp + kv0, 0, 0);
  }
  // Mask / bias of the tile.  Full tiles use the DMA; the partial last tile loads element by
  // element with a bounds check (a 16-byte DMA chunk that straddles the end of a [B, Sk]
  // row is range-checked as a whole and would read back as zeros).
  const bool tail = kv0 + 128 > Sk;
  if constexpr (HAS_BIAS) {
    if (wave == 0) {
      if (!tail) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, LDS_PTR(sAux), 16, (uint32_t)(kv0 * 4 + (lane & 31) * 16), 0,
                                                 0, 0);
      } else if (lane < 32) {
        v4f b4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = kv0 + 4 * lane + e;
          b4[e] = key < Sk ? bias_row[key] : 0.0f;
        }
        *reinterpret_cast<v4f*>(sAux + 16 * lane) = b4;
      }
    }
  }
  if constexpr (HAS_MASK) {
    if (wave == 1) {
      if (!tail) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(mrs, LDS_PTR(sAux + 1024), 16, (uint32_t)(kv0 + (lane & 7) * 16), 0,
                                                 0, 0);
      } else if (lane < 8) {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kv0 + 16 * lane + e;
          const uint32_t byte = key < Sk ? (uint32_t)mask_row[key] : 0u;
          w[e >> 2] |= byte << (8 * (e & 3));
        }
        *reinterpret_cast<v4i*>(sAux + 1024 + 16 * lane) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      }
    }
  }
}

template <int D, bool HAS_MASK, bool HAS_BIAS, bool DO_REPAIR>
struct AttnState {
  static constexpr int NDT = D / 32;  // O^T row tiles
  v16f o[NDT];
  v16f orep[DO_REPAIR ? NDT : 1];
  float m, l;
};

// Process one KV tile held in LDS.
template <int D, bool HAS_MASK, bool HAS_BIAS, bool DO_REPAIR>
__device__ __forceinline__ void attn_tile(const uint8_t* sK, const uint8_t* sV, const uint8_t* sAux,
                                          const v8i (&qf)[D / 64], float sq, float skj, int kv0, int Sk,
                                          float tau, int lane, AttnState<D, HAS_MASK, HAS_BIAS, DO_REPAIR>& st) {
  constexpr int NDT = D / 32;
  constexpr float NEG = -1.0e9f;
  const int g = lane >> 5;
  // ---- S^T = K Q^T (4 subtiles of 32 keys x 32 queries)
  v16f s[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[t][i] = 0.0f;
#pragma unroll
    for (int h = 0; h < D / 64; ++h) {
      const v8i kf = lds_read32<D>(sK, 32 * t + (lane & 31), D, D / 16, 4 * h + 2 * g);
      s[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf, qf[h], s[t], 0, 0, 0, 0, 0, 0);
    }
  }
  // ---- scale, bias, validity; s[t][i] is key 64(t/2) + 16(t%2) + 32g + i of the tile
  const bool full = (kv0 + 128 <= Sk) && !HAS_MASK && !HAS_BIAS;
  uint64_t validbits = ~0ull;  // bit 16t + i
  float rmax = NEG;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int kb = 64 * (t >> 1) + 16 * (t & 1) + 32 * g;
    float bias[16];
    if constexpr (HAS_BIAS) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const v4f b4 = *reinterpret_cast<const v4f*>(sAux + (kb + 4 * q4) * 4);
        bias[4 * q4 + 0] = b4[0]; bias[4 * q4 + 1] = b4[1]; bias[4 * q4 + 2] = b4[2]; bias[4 * q4 + 3] = b4[3];
      }
    }
    uint32_t mbytes[4] = {~0u, ~0u, ~0u, ~0u};
    if constexpr (HAS_MASK) {
      const v4i m4 = *reinterpret_cast<const v4i*>(sAux + 1024 + kb);
      mbytes[0] = m4[0]; mbytes[1] = m4[1]; mbytes[2] = m4[2]; mbytes[3] = m4[3];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = (s[t][i] * sq) * skj;
      if (!full) {
        bool ok = kv0 + kb + i < Sk;
        if constexpr (HAS_BIAS) {
          ok = ok && (bias[i] > -1.0e8f);
          v = v + bias[i] * 1.4426950408889634f;
        }
        if constexpr (HAS_MASK) ok = ok && (((mbytes[i >> 2] >> (8 * (i & 3))) & 0xffu) != 0u);
        if (!ok) {
          v = NEG;
          validbits &= ~(1ull << (16 * t + i));
        }
      }
      s[t][i] = v;
      rmax = fmaxf(rmax, v);
    }
  }
  rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
  // ---- lazy max
  const float m_old = st.m;
  const float m_new = (rmax > m_old + 8.0f || m_old == NEG) ? rmax : m_old;
  const float alpha = __builtin_amdgcn_exp2f(m_old - m_new);
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // wave-uniform: skip when no row moved
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) st.o[dt][i] *= alpha;
      if constexpr (DO_REPAIR) {
#pragma unroll
        for (int i = 0; i < 16; ++i) st.orep[dt][i] *= alpha;
      }
    }
    st.l *= alpha;
  }
  st.m = m_new;
  // ---- exp2-free P codes, row sum, packing into the PV B operand
  const float cst = 56.0f - 8.0f * m_new;
  v8i pf[2];
  float lsum = 0.0f;
  float pexact[DO_REPAIR ? 64 : 1];
  float papx[DO_REPAIR ? 64 : 1];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * w4 + e;
        const float bits = __builtin_fmaf(s[t][i], 8.0f, cst);
        const bool valid = (validbits >> (16 * t + i)) & 1ull;
        const float code = (bits < 8.0f || !valid) ? 0.0f : fminf(fmaxf(__builtin_rintf(bits), 0.0f), 126.0f);
        word = __builtin_amdgcn_cvt_pk_u8_f32(code, e, word);
        const uint32_t ci = (uint32_t)code;
        const float p = ci ? __uint_as_float((ci << 20) + 0x3C000000u) : 0.0f;
        lsum += p;
        if constexpr (DO_REPAIR) {
          papx[16 * t + i] = p;
          pexact[16 * t + i] = valid ? __builtin_amdgcn_exp2f(s[t][i] - m_new) : 0.0f;
        }
      }
      pf[t >> 1][4 * (t & 1) + w4] = (int)word;
    }
  }
  st.l += lsum;
  // ---- O^T += V^T P^T
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const v8i vf = lds_read32<D>(sV, 32 * dt + (lane & 31), 128, 8, 4 * kh + 2 * g);
      st.o[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf[kh], st.o[dt], 0, 0, 0, 0, 0, 0);
    }
  }
  if constexpr (DO_REPAIR) {
    // delta = exp2(S - m) - P where P >= tau; O_r^T += bf16(V^T) bf16(delta^T) over 16-key
    // chunks: chunk (t, u) gives lane group g the 8 keys 64(t/2) + 16(t%2) + 32g + 8u + 0..7.
    float dsum = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        v8bf db;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 16 * t + 8 * u + e;
          const float d = (papx[i] >= tau) ? (pexact[i] - papx[i]) : 0.0f;
          dsum += d;
          db[e] = __builtin_bit_cast(__bf16, (unsigned short)f32_to_bf16_bits(d));
        }
        const int key0 = 64 * (t >> 1) + 16 * (t & 1) + 32 * g + 8 * u;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int row = 32 * dt + (lane & 31);
          const int c = key0 >> 4;
          const uint8_t* src = sV + row * 128 + ((c ^ (row & 7)) << 4) + (key0 & 15);
          const v2i raw = *reinterpret_cast<const v2i*>(src);
          v8bf vb;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t byte = ((uint32_t)raw[e >> 2] >> (8 * (e & 3))) & 0xffu;
            // e4m3 -> bf16 is exact: rebias the exponent (7 -> 127) and widen the mantissa.
            const uint32_t sgn = (byte & 0x80u) << 8, mag = byte & 0x7fu;
            uint32_t bits;
            if (mag >= 8u) {
              bits = sgn | ((mag + (120u << 3)) << 4);
            } else {  // subnormal: mag * 2^-9
              const float f = (float)mag * 0.001953125f;
              bits = sgn | (__float_as_uint(f) >> 16);
            }
            vb[e] = __builtin_bit_cast(__bf16, (unsigned short)bits);
          }
          st.orep[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, db, st.orep[dt], 0, 0, 0);
        }
      }
    }
    st.l += dsum;
  }
}

template <int D, bool HAS_MASK, bool HAS_BIAS, bool DO_REPAIR, int ODT>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const uint8_t* __restrict__ q8, const uint8_t* __restrict__ k8,
                                                       const uint8_t* __restrict__ v8t, const float* __restrict__ sq,
                                                       const float* __restrict__ sk, const float* __restrict__ sv,
                                                       const uint8_t* __restrict__ key_mask,
                                                       const float* __restrict__ key_bias, float tau,
                                                       void* __restrict__ out, int64_t os_b, int64_t os_h,
                                                       int64_t os_s, int64_t os_d, int H, int Sq, int Sk) {
  typedef AttnTile<D> T;
  constexpr int NDT = D / 32;
  __shared__ __attribute__((aligned(1024))) uint8_t sK0[T::KB];
  __shared__ __attribute__((aligned(1024))) uint8_t sV0[T::VB];
  __shared__ __attribute__((aligned(1024))) uint8_t sA0[(HAS_MASK || HAS_BIAS) ? T::AUXB : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t sK1[T::KB];
  __shared__ __attribute__((aligned(1024))) uint8_t sV1[T::VB];
  __shared__ __attribute__((aligned(1024))) uint8_t sA1[(HAS_MASK || HAS_BIAS) ? T::AUXB : 16];

  const int I = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int nq = gridDim.x;
  const int nk = (Sk + 127) / 128;
  const int Sqp = nq * 128, Skp = nk * 128;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = lane >> 5;

  // ---- Q fragments (B operand of S^T): query row q0 + lane%32, bytes [64h + 32g, +32)
  const int qrow = I * 128 + wave * 32 + (lane & 31);
  v8i qf[D / 64];
  {
    const uint8_t* qp = q8 + ((int64_t)bh * Sqp + qrow) * D + 32 * g;
#pragma unroll
    for (int hh = 0; hh < D / 64; ++hh) {
      const v4i lo = *reinterpret_cast<const v4i*>(qp + 64 * hh);
      const v4i hi = *reinterpret_cast<const v4i*>(qp + 64 * hh + 16);
      qf[hh][0] = lo[0]; qf[hh][1] = lo[1]; qf[hh][2] = lo[2]; qf[hh][3] = lo[3];
      qf[hh][4] = hi[0]; qf[hh][5] = hi[1]; qf[hh][6] = hi[2]; qf[hh][7] = hi[3];
    }
  }
  const float sqI = sq[(int64_t)bh * nq + I];
  const float* skh = sk + (int64_t)bh * nk;

  // ---- DMA descriptors and per-lane offsets
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(k8 + (int64_t)bh * Skp * D), 0, Skp * D, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(v8t + (int64_t)bh * D * Skp), 0, D * Skp, 0x00020000);
  __amdgpu_buffer_rsrc_t brs = krs, mrs = krs;
  if constexpr (HAS_BIAS)
    brs = __builtin_amdgcn_make_buffer_rsrc((void*)(key_bias + (int64_t)b * Sk), 0, Sk * 4, 0x00020000);
  if constexpr (HAS_MASK)
    mrs = __builtin_amdgcn_make_buffer_rsrc((void*)(key_mask + (int64_t)b * Sk), 0, Sk, 0x00020000);
  const float* brow = HAS_BIAS ? key_bias + (int64_t)b * Sk : nullptr;
  const uint8_t* mrow = HAS_MASK ? key_mask + (int64_t)b * Sk : nullptr;
  uint32_t k_lane;
  if constexpr (D == 128) {
    // lane i: LDS row 8J + i/8, phys chunk i%8 -> logical (i%8) ^ (i/8); key part of the lane
    k_lane = (uint32_t)((32 * ((lane >> 5) & 1) + ((lane >> 3) & 3)) * D + (((lane & 7) ^ (lane >> 3)) << 4));
  } else {
    // 64-byte rows: lane i: LDS row 16J + i/4, phys chunk i%4 -> logical (i%4) ^ ((i/4)&3)
    const int rr = lane >> 2;  // row within the 16-row instruction, R = 16(J&1) + rr
    k_lane = (uint32_t)((32 * ((rr >> 2) & 1) + 4 * (rr >> 3) + (rr & 3)) * D +
                        (((lane & 3) ^ (rr & 3)) << 4));
  }
  const uint32_t v_lane = (uint32_t)((lane >> 3) * Skp + (((lane & 7) ^ (lane >> 3)) << 4));
  constexpr int PER_TILE = T::K_INSTR + T::V_INSTR;

  AttnState<D, HAS_MASK, HAS_BIAS, DO_REPAIR> st;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      st.o[dt][i] = 0.0f;
      if constexpr (DO_REPAIR) st.orep[dt][i] = 0.0f;
    }
  st.m = -1.0e9f;
  st.l = 0.0f;

  const int j0 = (int)(((int64_t)I * nk) / nq);
  auto jof = [&](int i) { int j = j0 + i; return j >= nk ? j - nk : j; };

  attn_dma<D, HAS_MASK, HAS_BIAS>(krs, vrs, brs, mrs, sK0, sV0, sA0, k_lane, v_lane, wave, lane, jof(0) * 128, Skp, Sk, brow, mrow);
  int i = 0;
  for (; i + 2 < nk; i += 2) {
    const int ja = jof(i), jb = jof(i + 1);
    attn_dma<D, HAS_MASK, HAS_BIAS>(krs, vrs, brs, mrs, sK1, sV1, sA1, k_lane, v_lane, wave, lane, jb * 128, Skp, Sk, brow, mrow);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_TILE) : "memory");
    attn_barrier();
    attn_tile<D, HAS_MASK, HAS_BIAS, DO_REPAIR>(sK0, sV0, sA0, qf, sqI, skh[ja], ja * 128, Sk, tau, lane, st);
    attn_barrier();
    attn_dma<D, HAS_MASK, HAS_BIAS>(krs, vrs, brs, mrs, sK0, sV0, sA0, k_lane, v_lane, wave, lane, jof(i + 2) * 128,
                                    Skp, Sk, brow, mrow);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_TILE) : "memory");
    attn_barrier();
    attn_tile<D, HAS_MASK, HAS_BIAS, DO_REPAIR>(sK1, sV1, sA1, qf, sqI, skh[jb], jb * 128, Sk, tau, lane, st);
    attn_barrier();
  }
  const bool two_left = i + 1 < nk;
  if (two_left) {
    const int ja = jof(i), jb = jof(i + 1);
    attn_dma<D, HAS_MASK, HAS_BIAS>(krs, vrs, brs, mrs, sK1, sV1, sA1, k_lane, v_lane, wave, lane, jb * 128, Skp, Sk, brow, mrow);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_TILE) : "memory");
    attn_barrier();
    attn_tile<D, HAS_MASK, HAS_BIAS, DO_REPAIR>(sK0, sV0, sA0, qf, sqI, skh[ja], ja * 128, Sk, tau, lane, st);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  attn_barrier();
  {
    const int jl = jof(two_left ? i + 1 : i);
    attn_tile<D, HAS_MASK, HAS_BIAS, DO_REPAIR>(two_left ? sK1 : sK0, two_left ? sV1 : sV0, two_left ? sA1 : sA0, qf,
                                                sqI, skh[jl], jl * 128, Sk, tau, lane, st);
  }

  // ---- epilogue: O = (O + O_r) * sv / max(l, 1e-12); lane holds query qrow, channels
  // 32 dt + 8 (i/4) + 4 g + i%4
  const float l = st.l + __shfl_xor(st.l, 32, 64);
  if (qrow >= Sq) return;
  const float den = fmaxf(l, 1.0e-12f);
  const float* svh = sv + (int64_t)bh * D;
  char* obase = static_cast<char*>(out) + ((int64_t)b * os_b + (int64_t)h * os_h + (int64_t)qrow * os_s) * 2;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d0 = 32 * dt + 8 * q4 + 4 * g;
      uint32_t ob[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float acc = st.o[dt][4 * q4 + e];
        if constexpr (DO_REPAIR) acc += st.orep[dt][4 * q4 + e];
        const float v = __fdiv_rn(acc * svh[d0 + e], den);
        ob[e] = ODT == MXF8_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
      }
      uint16_t* dst = reinterpret_cast<uint16_t*>(obase) + (int64_t)d0 * os_d;
      if (os_d == 1) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(ob[0] | (ob[1] << 16), ob[2] | (ob[3] << 16));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(int64_t)e * os_d] = (uint16_t)ob[e];
      }
    }
  }
}

template <int D, bool M_, bool B_, bool R_, int ODT>
static void launch_attn(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t, const float* sq, const float* sk,
                        const float* sv, const uint8_t* km, const float* kb, float tau, void* out,
                        const int64_t os[4], int64_t B, int64_t H, int64_t Sq, int64_t Sk, hipStream_t st) {
  dim3 grid((unsigned)cdiv(Sq, 128), (unsigned)(B * H));
  attn_fwd_kernel<D, M_, B_, R_, ODT><<<grid, 256, 0, st>>>(q8, k8, v8t, sq, sk, sv, km, kb, tau, out, os[0], os[1],
                                                            os[2], os[3], (int)H, (int)Sq, (int)Sk);
}

template <int D, int ODT>
static void attn_dispatch_flags(bool hm, bool hb, bool rep, const uint8_t* q8, const uint8_t* k8,
                                const uint8_t* v8t, const float* sq, const float* sk, const float* sv,
                                const uint8_t* km, const float* kb, float tau, void* out, const int64_t os[4],
                                int64_t B, int64_t H, int64_t Sq, int64_t Sk, hipStream_t st) {
#define MXF8_ATTN_CASE(M_, B_, R_)                                                                       \
  if (hm == M_ && hb == B_ && rep == R_) {                                                               \
    launch_attn<D, M_, B_, R_, ODT>(q8, k8, v8t, sq, sk, sv, km, kb, tau, out, os, B, H, Sq, Sk, st); \
    return;                                                                                              \
  }
  MXF8_ATTN_CASE(false, false, false)
  MXF8_ATTN_CASE(true, false, false)
  MXF8_ATTN_CASE(false, true, false)
  MXF8_ATTN_CASE(true, true, false)
  MXF8_ATTN_CASE(false, false, true)
  MXF8_ATTN_CASE(true, false, true)
  MXF8_ATTN_CASE(false, true, true)
  MXF8_ATTN_CASE(true, true, true)
#undef MXF8_ATTN_CASE
}


// One translation unit per (D, output dtype) instantiates attn_dispatch_flags.
#define MXF8_ATTN_DECL(D_, ODT_)                                                                             \
  void attn_launch_##D_##_##ODT_(bool hm, bool hb, bool rep, const uint8_t* q8, const uint8_t* k8,         \
                                 const uint8_t* v8t, const float* sq, const float* sk, const float* sv,     \
                                 const uint8_t* km, const float* kb, float tau, void* out,                  \
                                 const int64_t os[4], int64_t B, int64_t H, int64_t Sq, int64_t Sk,         \
                                 hipStream_t st)
MXF8_ATTN_DECL(128, 0);
MXF8_ATTN_DECL(128, 1);
MXF8_ATTN_DECL(64, 0);
MXF8_ATTN_DECL(64, 1);

}  // namespace mxf8
