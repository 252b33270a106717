// FP8 flash-attention forward for gfx950 (non-causal; optional per-key mask / bias).
//
// Algorithm (kernels/fp8_attention.py:215-297, BLOCK_M = BLOCK_N = 128): per (b, h, Q tile
// I of 128 rows) the KV tiles are visited in the staggered order j = (j0 + i) % nk with
// j0 = I*nk/nq; scores are in the log2 domain S = (Q8 K8^T) * sq * sk (+ bias * log2 e);
// the row max m is lazy (it moves to the tile max only when that exceeds m + 8, or while
// m is still -1e9); P is produced without exp2 as the e4m3 code rint(8 S + 56 - 8 m)
// (0 below 8); l += sum(P); O += P V; with repair_tau >= 0, exp2(S - m) - P is added for
// codes >= tau through bf16.  Output = O * sv / max(l, 1e-12).
//
// Mapping to CDNA4.  A workgroup (4 waves) owns one Q tile; wave w owns its 32 rows, and
// two workgroups share a CU (the kernel is register-limited to 256 VGPRs per lane) so that
// one wave's softmax (VALU) overlaps the other's matrix products on each SIMD.  The
// kernel computes the TRANSPOSED score tile S^T = K Q^T with v_mfma_f32_32x32x64_f8f6f4:
// in the 32x32 accumulator layout lane l holds query column l%32, so every per-query
// statistic is lane-local (plus one exchange with lane l^32).  The K rows of each 32-key
// subtile are fed to the MFMA in a permuted order chosen so that the accumulator
// registers, packed 4 codes per dword, ARE the B operand of the PV MFMA (O^T = V^T P^T)
// with V^T read as contiguous 32-byte runs of a v8t row: no cross-lane shuffles between
// the two products.  The row sums l come from the matrix cores too: one more MFMA per
// 64 keys with an all-ones A operand.  K and V^T tiles (and the mask / bias of the tile)
// are copied global -> LDS by the direct-to-LDS DMA into two buffers; one barrier per
// tile both publishes tile i and retires the buffer that tile i+1 is loaded into.
//
// Per score the VALU does half a 3-input max, two FMAs (8 S + 56 - 8 m straight from the
// fp32 dot product with the per-tile constant 8 sq sk, and the same shifted and scaled
// for the flush test), a min and a rounding byte pack.  Folding sq * sk into one constant
// rounds 8 S once instead of twice; the row max that drives the lazy-max policy is still
// computed exactly as (max * sq) * sk.
#pragma once

#include "common.h"

namespace mxf8 {

constexpr float kAttnNeg = -1.0e9f;

__device__ __forceinline__ void attn_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Key (within a 128-key tile) of accumulator row R of score subtile t.  Subtile t covers
// keys 64(t/2) + 16(t%2) + {0..15, 32..47}; register i of lane group g of subtile t then
// holds key 64(t/2) + 32g + 16(t%2) + i, i.e. the byte order of the PV B operand.
__host__ __device__ constexpr int key_of_row(int t, int R) {
  return 64 * (t >> 1) + 16 * (t & 1) + 32 * ((R >> 2) & 1) + 4 * (R >> 3) + (R & 3);
}

template <int D, bool AUX>
struct AttnTile {
  static constexpr int KB = 128 * D;             // K tile bytes (128 keys x D)
  static constexpr int VB = D * 128;             // V^T tile bytes (D rows x 128 keys)
  static constexpr int AUXB = AUX ? 2048 : 0;    // bias (1 KB) + mask (1 KB)
  static constexpr int BUF = KB + VB + AUXB;     // one LDS buffer
  static constexpr int CPRK = D / 16;            // 16-byte chunks per K row
  static constexpr int K_INSTR = KB / 1024 / 4;  // 1 KB DMA instructions per wave
  static constexpr int V_INSTR = VB / 1024 / 4;
};

// 32 bytes = logical chunks chunk0, chunk0 + 1 of `row` of a swizzled tile.
template <int ROW_BYTES>
__device__ __forceinline__ v8i lds_read32(const uint8_t* tile, int row, int chunk0) {
  const int sw = lds_swz<ROW_BYTES>(row);
  const v4i lo = *reinterpret_cast<const v4i*>(tile + row * ROW_BYTES + ((chunk0 ^ sw) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(tile + row * ROW_BYTES + (((chunk0 + 1) ^ sw) << 4));
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// DMA one KV tile (keys [kv0, kv0 + 128)) of head bh into the LDS buffer `buf`.
template <int D, bool HAS_MASK, bool HAS_BIAS>
__device__ __forceinline__ void attn_dma(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                         __amdgpu_buffer_rsrc_t brs, __amdgpu_buffer_rsrc_t mrs, uint8_t* buf,
                                         const uint32_t (&k_lane)[2], const uint32_t (&v_lane)[2], int wave, int lane,
                                         int kv0, int Skp,
                                         int Sk, const float* bias_row, const uint8_t* mask_row) {
  typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
  uint8_t* sK = buf;
  uint8_t* sV = buf + T::KB;
  uint8_t* sAux = buf + T::KB + T::VB;
#pragma unroll
  for (int j = 0; j < T::K_INSTR; ++j) {
    const int J = wave * T::K_INSTR + j;
    // LDS rows of instruction J: accumulator row R of subtile t = R/32 loads key key_of_row.
    int ubase;
    if constexpr (D == 128) {
      const int t = J >> 2;
      ubase = 64 * (t >> 1) + 16 * (t & 1) + 4 * (J & 3);
    } else {
      const int t = J >> 1;
      ubase = 64 * (t >> 1) + 16 * (t & 1) + 8 * (J & 1);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, LDS_PTR(sK + J * 1024), 16, k_lane[j & 1], (kv0 + ubase) * D, 0,
                                             0);
  }
#pragma unroll
  for (int j = 0; j < T::V_INSTR; ++j) {
    const int J = wave * T::V_INSTR + j;  // V^T rows [8J, 8J + 8)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, LDS_PTR(sV + J * 1024), 16, v_lane[j & 1], 8 * J * Skp + kv0, 0,
                                             0);
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

template <int D, bool DO_REPAIR>
struct AttnState {
  static constexpr int NDT = D / 32;  // O^T row tiles
  v16f o[NDT];
  v16f orep[DO_REPAIR ? NDT : 1];
  v16f lacc;     // every register holds the running sum of P codes of the lane's query
  float m;       // lazy row max (log2 domain)
  float ldelta;  // repair: running sum of the exact-minus-code corrections (lane's keys)
};

// e4m3 value of a P code (codes are 0 or in [8, 126], i.e. zero or normal).
__device__ __forceinline__ float p_value(uint32_t code) {
  return code ? __uint_as_float((code << 20) + 0x3C000000u) : 0.0f;
}

// Process one KV tile held in LDS buffer `buf`.
template <int D, bool HAS_MASK, bool HAS_BIAS, bool DO_REPAIR>
__device__ __forceinline__ void attn_tile(const uint8_t* buf, const v8i (&qf)[D / 64], float sq, float skj, int kv0,
                                          int Sk, float tau, int lane, AttnState<D, DO_REPAIR>& st) {
  typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
  constexpr int NDT = D / 32;
  constexpr float LOG2E_F = 1.4426950408889634f;
  const uint8_t* sK = buf;
  const uint8_t* sV = buf + T::KB;
  const uint8_t* sAux = buf + T::KB + T::VB;
  const int g = lane >> 5;

  // ---- S^T = K Q^T (4 subtiles of 32 keys x 32 queries); s[t][i] is key 64(t/2) + 32g + 16(t%2) + i
  v16f s[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[t][i] = 0.0f;
#pragma unroll
    for (int h = 0; h < D / 64; ++h) {
      const v8i kf = lds_read32<D>(sK, 32 * t + (lane & 31), 4 * h + 2 * g);
      s[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kf, qf[h], s[t], 0, 0, 0, 0, 0, 0);
    }
  }

  // ---- scores of invalid keys become -inf; with a bias, S is formed explicitly
  const bool partial = kv0 + 128 > Sk;
  if (HAS_MASK || HAS_BIAS || partial) {
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
        bool ok = kv0 + kb + i < Sk;
        float v = s[t][i];
        if constexpr (HAS_BIAS) {
          ok = ok && (bias[i] > -1.0e8f);
          v = (v * sq) * skj + bias[i] * LOG2E_F;
        }
        if constexpr (HAS_MASK) ok = ok && (((mbytes[i >> 2] >> (8 * (i & 3))) & 0xffu) != 0u);
        s[t][i] = ok ? v : -INFINITY;
      }
    }
  }

  // ---- row max (exactly the reference's fp32 S max: x -> (x * sq) * sk is monotonic)
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[t][i]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float rmax = fmaxf(HAS_BIAS ? mx : (mx * sq) * skj, kAttnNeg);

  // ---- lazy max
  const float m_old = st.m;
  const float m_new = (rmax > m_old + 8.0f || m_old == kAttnNeg) ? rmax : m_old;
  if (__builtin_amdgcn_ballot_w64(m_new != m_old)) {  // wave-uniform: skip when no row moved
    const float alpha = __builtin_amdgcn_exp2f(m_old - m_new);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) st.o[dt][i] *= alpha;
      if constexpr (DO_REPAIR) {
#pragma unroll
        for (int i = 0; i < 16; ++i) st.orep[dt][i] *= alpha;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) st.lacc[i] *= alpha;
    if constexpr (DO_REPAIR) st.ldelta *= alpha;
  }
  st.m = m_new;

  // ---- exp2-free P codes: code = bits < 8 ? 0 : rint(bits), bits = 8 S + 56 - 8 m.  bits
  // never exceeds 8 * 8 + 56 = 120 (the lazy max keeps S <= m + 8), so the reference's
  // clamp to [0, 126] is inactive.  v_cvt_pk_u8_f32 rounds to nearest even and saturates
  // negative inputs to 0, so it performs rint itself; the flush below 8 is
  // min(bits, (bits - 8) * 2^24), negative exactly when bits < 8 and equal to bits when
  // bits >= 8 + 2^-21.  Invalid keys carry S = -inf and flush to 0.
  const float cst = 56.0f - 8.0f * m_new;
  const float c8 = HAS_BIAS ? 8.0f : (8.0f * sq) * skj;
  const float c8f = c8 * 16777216.0f;
  const float cstf = (48.0f - 8.0f * m_new) * 16777216.0f;
  v8i pf[2];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float bits = __builtin_fmaf(s[t][4 * w4 + e], c8, cst);
        const float flush = __builtin_fmaf(s[t][4 * w4 + e], c8f, cstf);
        word = __builtin_amdgcn_cvt_pk_u8_f32(fminf(bits, flush), e, word);
      }
      pf[t >> 1][4 * (t & 1) + w4] = (int)word;
    }
  }

  // ---- O^T += V^T P^T, l += 1^T P^T
  const v8i ones = {0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838};
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const v8i vf = lds_read32<128>(sV, 32 * dt + (lane & 31), 4 * kh + 2 * g);
      st.o[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf[kh], st.o[dt], 0, 0, 0, 0, 0, 0);
    }
    st.lacc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ones, pf[kh], st.lacc, 0, 0, 0, 0, 0, 0);
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
          const int i = 8 * u + e;
          const uint32_t code = ((uint32_t)pf[t >> 1][4 * (t & 1) + (i >> 2)] >> (8 * (i & 3))) & 0xffu;
          const float papx = p_value(code);
          const float S = HAS_BIAS ? s[t][i] : (s[t][i] * sq) * skj;
          const float pexact = __builtin_amdgcn_exp2f(S - m_new);  // invalid keys: S = -inf -> 0
          const float d = (papx >= tau) ? (pexact - papx) : 0.0f;
          dsum += d;
          db[e] = __builtin_bit_cast(__bf16, (unsigned short)f32_to_bf16_bits(d));
        }
        const int key0 = 64 * (t >> 1) + 16 * (t & 1) + 32 * g + 8 * u;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int row = 32 * dt + (lane & 31);
          const int c = key0 >> 4;
          const uint8_t* src = sV + row * 128 + ((c ^ lds_swz<128>(row)) << 4) + (key0 & 15);
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
    st.ldelta += dsum;
  }
}

// Register budget: 256 VGPRs per lane (two waves per SIMD) for the plain kernel; the
// repair variant keeps S, codes and the correction accumulator live and runs one wave.
template <bool DO_REPAIR>
struct AttnOccupancy {
  static constexpr int waves = DO_REPAIR ? 1 : 2;
};

template <int D, bool HAS_MASK, bool HAS_BIAS, bool DO_REPAIR, int ODT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(AttnOccupancy<DO_REPAIR>::waves)))
void attn_fwd_kernel(const uint8_t* __restrict__ q8, const uint8_t* __restrict__ k8, const uint8_t* __restrict__ v8t,
                     const float* __restrict__ sq, const float* __restrict__ sk, const float* __restrict__ sv,
                     const uint8_t* __restrict__ key_mask, const float* __restrict__ key_bias, float tau,
                     void* __restrict__ out, int64_t os_b, int64_t os_h, int64_t os_s, int64_t os_d, int H, int Sq,
                     int Sk, int nq) {
  typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
  constexpr int NDT = D / 32;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * T::BUF];

  // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a contiguous range of
  // (head, Q tile) ids so that the workgroups resident on one XCD are consecutive Q tiles
  // of one head, whose staggered KV sweeps overlap and share that XCD's L2.
  int bh, I;
  {
    const int total = gridDim.x, L = blockIdx.x;
    const int q = total >> 3, r = total & 7, x = L & 7, kk = L >> 3;
    const int id = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + kk;
    bh = id / nq;
    I = id - bh * nq;
  }
  const int b = bh / H, h = bh - (bh / H) * H;
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
  // Per-lane DMA offsets.  A 1 KB DMA instruction J fills LDS bytes [1024 J, +1024): lane i
  // writes 16 bytes at row 8J + i/8 (128-byte rows) or 16J + i/4 (64-byte rows), physical
  // chunk i%8 (i%4), which must hold logical chunk phys ^ lds_swz(row); for 128-byte rows
  // that depends on the parity of J, hence one offset per parity.
  uint32_t k_lane[2], v_lane[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int vrow = 8 * par + (lane >> 3);  // row of a 128-byte-row tile, mod 16
    const uint32_t chunk128 = (uint32_t)(((lane & 7) ^ lds_swz<128>(vrow)) << 4);
    v_lane[par] = (uint32_t)((lane >> 3) * Skp) + chunk128;
    if constexpr (D == 128) {
      // key of LDS row 8J + i/8 relative to the instruction's first key (key_of_row)
      k_lane[par] = (uint32_t)((32 * ((lane >> 5) & 1) + ((lane >> 3) & 3)) * D) + chunk128;
    } else {
      const int rr = lane >> 2;  // row within the 16-row instruction, R = 16(J&1) + rr
      k_lane[par] = (uint32_t)((32 * ((rr >> 2) & 1) + 4 * (rr >> 3) + (rr & 3)) * D +
                               (((lane & 3) ^ lds_swz<64>(rr)) << 4));
    }
  }

  AttnState<D, DO_REPAIR> st;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      st.o[dt][i] = 0.0f;
      if constexpr (DO_REPAIR) st.orep[dt][i] = 0.0f;
    }
#pragma unroll
  for (int i = 0; i < 16; ++i) st.lacc[i] = 0.0f;
  st.m = kAttnNeg;
  st.ldelta = 0.0f;

  const int j0 = (int)(((int64_t)I * nk) / nq);
  attn_dma<D, HAS_MASK, HAS_BIAS>(krs, vrs, brs, mrs, smem, k_lane, v_lane, wave, lane, j0 * 128, Skp, Sk, brow,
                                  mrow);
  int j = j0;
  for (int i = 0; i < nk; ++i) {
    // Tile i is the only DMA in flight; after the barrier every wave has finished tile
    // i-1, so its buffer can take tile i+1 while tile i is computed.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    attn_barrier();
    const int jn = j + 1 == nk ? 0 : j + 1;
    if (i + 1 < nk)
      attn_dma<D, HAS_MASK, HAS_BIAS>(krs, vrs, brs, mrs, smem + ((i + 1) & 1) * T::BUF, k_lane, v_lane, wave, lane,
                                      jn * 128, Skp, Sk, brow, mrow);
    attn_tile<D, HAS_MASK, HAS_BIAS, DO_REPAIR>(smem + (i & 1) * T::BUF, qf, sqI, skh[j], j * 128, Sk, tau, lane,
                                                st);
    j = jn;
  }

  // ---- epilogue: O = (O + O_r) * sv / max(l, 1e-12); lane holds query qrow, channels
  // 32 dt + 8 (i/4) + 4 g + i%4
  if (qrow >= Sq) return;
  float l = st.lacc[0];
  if constexpr (DO_REPAIR) l += st.ldelta + __shfl_xor(st.ldelta, 32, 64);
  const float den = fmaxf(l, 1.0e-12f);
  const float* svh = sv + (int64_t)bh * D;
  char* obase = static_cast<char*>(out) + ((int64_t)b * os_b + (int64_t)h * os_h + (int64_t)qrow * os_s) * 2;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d0 = 32 * dt + 8 * q4 + 4 * g;
      const v4f sv4 = *reinterpret_cast<const v4f*>(svh + d0);
      uint32_t ob[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float acc = st.o[dt][4 * q4 + e];
        if constexpr (DO_REPAIR) acc += st.orep[dt][4 * q4 + e];
        const float v = __fdiv_rn(acc * sv4[e], den);
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
  const int64_t nq = cdiv(Sq, 128);
  dim3 grid((unsigned)(nq * B * H));
  attn_fwd_kernel<D, M_, B_, R_, ODT><<<grid, 256, 0, st>>>(q8, k8, v8t, sq, sk, sv, km, kb, tau, out, os[0], os[1],
                                                            os[2], os[3], (int)H, (int)Sq, (int)Sk, (int)nq);
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
