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
// Mapping to CDNA4.  A workgroup of 4 waves owns one Q tile;
// wave w owns its 32 rows.  The kernels compute the TRANSPOSED score tile S^T = K Q^T with
// v_mfma_f32_32x32x64_f8f6f4: in the 32x32 accumulator layout lane l holds query column
// l%32, so every per-query statistic is lane-local (plus one exchange with lane l^32).  The
// K rows of each 32-key subtile are fed to the MFMA in a permuted order chosen so that the
// accumulator registers, packed 4 codes per dword, ARE the B operand of the PV MFMA
// (O^T = V^T P^T) with V^T read as contiguous 32-byte runs of a v8t row: no cross-lane
// shuffles between the two products.  The row sums l come from the matrix cores too: one
// v_mfma_f32_16x16x128_f8f6f4 per 64 keys that reads the P fragment as its B operand and
// a lane-constant 0/1 selector as A (AttnFragOfs::rowsum_sel).  K and V^T tiles (and the
// mask / bias of the tile) are copied global -> LDS by the direct-to-LDS DMA.
//
// Per score the VALU does half a 3-input max and three FMAs ((8 S + 56 - 8 m) / 8 straight
// from the fp32 dot product with the per-tile constant sq sk; the flush test as a clamped
// FMA; rounding to an integer code by adding 1.5 * 2^20), plus three quarters of a byte
// permute to pack the codes.  Folding sq * sk into one constant rounds 8 S once instead of
// twice; the row max that drives the lazy-max policy is still computed exactly as
// (max * sq) * sk.
//
// The repair correction delta = exp2(S - m) - P (where P >= tau) is formed from the same
// bits and split into two e4m3 parts of 8 delta that the PV products multiply with the V^T
// fragments already loaded for P V, at the MFMA's E8M0 block scale 2^-3; their row sums
// join l on the row-sum product.  The corrections accumulate into O itself (the reference
// keeps them in a second accumulator and adds the two at the end).
//
// One workgroup per Q tile processes one KV tile at a time: S = QK^T, codes, PV.  Two
// workgroups share a CU (the kernel fits 256 registers), so one wave's softmax overlaps
// the other's matrix products on each SIMD.  Each run of matrix products fetches its LDS
// fragments three products ahead.
#pragma once

#include <type_traits>

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
  static constexpr int K_INSTR = KB / 1024 / 4;  // 1 KB DMA instructions per wave
  static constexpr int V_INSTR = VB / 1024 / 4;
};

// Workgroups are dealt to the 8 XCDs round-robin; give each XCD a contiguous range of
// work items so that the workgroups resident on one XCD are consecutive Q tiles of one
// head, whose staggered KV sweeps overlap and share that XCD's L2.
__device__ __forceinline__ int xcd_linear_id(int L, int total) {
  const int q = total >> 3, r = total & 7, x = L & 7, kk = L >> 3;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + kk;
}

// 16-bit query for the fused Q quantizer: element (b, h, s, d) at q + b sb + h sh + s ss + d.
struct AttnQ16 {
  const uint16_t* q;
  int64_t sb, sh, ss;
  float c;        // softmax scale * log2(e)
  float* sq_out;  // [B, H, ceil(Sq / 128)] or null
};

// The Q block maximum of one 4-wave group, exchanged through LDS without a workgroup
// barrier (attn_fwd_resident_kernel): wave w of the group writes its maximum of round n to
// val[n & 1][w] and then n to tag[w]; a wave reads the four maxima once every tag has
// reached n.  A wave's LDS accesses take effect in issue order, so a tag never runs ahead
// of its value.  A value slot is written again at round n + 2, which its writer reaches only
// after the round n + 1 tags of all four waves, each written after that wave's round n read.
struct AttnGroupX {
  int tag[4];
  float val[2][4];
};

// Rounds a wave polls the tags before it gives up and goes on with the values it sees
// (with s_sleep 1, about 64 cycles each: some 0.2 s).  The four waves of a group go through
// the same rounds, so this bound is never reached; it keeps a wave from spinning forever.
constexpr int kAttnGroupXSpin = 1 << 22;

__device__ __forceinline__ void attn_group_publish(float amax, AttnGroupX* x, int wave, int round, int lane) {
  volatile int* tag = x->tag;
  volatile float* val = x->val[round & 1];
  if (lane == 0) {
    val[wave] = amax;
    tag[wave] = round;
  }
}

// The group's maximum of round `round`, once all four waves have published it.
__device__ __forceinline__ float attn_group_gather(AttnGroupX* x, int round) {
  volatile int* tag = x->tag;
  volatile float* val = x->val[round & 1];
  for (int it = 0; it < kAttnGroupXSpin; ++it) {
    const int t = __builtin_amdgcn_readfirstlane(min(min(tag[0], tag[1]), min(tag[2], tag[3])));
    if (t >= round) break;
    __builtin_amdgcn_s_sleep(1);
  }
  return fmaxf(fmaxf(val[0], val[1]), fmaxf(val[2], val[3]));
}

// Per-workgroup constants of a (b, h, Q tile) work item.  QF: the Q fragments are
// quantized by the workgroup from 16-bit Q (quant_q) instead of read from q8 / sq.
template <int D, bool HAS_MASK, bool HAS_BIAS, bool QF = false>
struct AttnCtx {
  int b, h, bh, I, nk, Skp, wave, lane, qrow;
  float sqI;
  const float* skh;
  v8i qf[D / 64];
  __amdgpu_buffer_rsrc_t krs, vrs, brs, mrs;
  const float* brow;
  const uint8_t* mrow;
  uint32_t k_lane[2], v_lane[2];

  // Work item id = bh * nq + I (head, Q tile); wave = the wave's index within the 4 waves
  // that own the Q tile.
  __device__ __forceinline__ AttnCtx(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t, const float* sq,
                                     const float* sk, const uint8_t* key_mask, const float* key_bias, int H, int Sk,
                                     int nq, int id, int wave_, int lane_) {
    bh = id / nq;
    I = id - bh * nq;
    b = bh / H;
    h = bh - b * H;
    nk = (Sk + 127) / 128;
    const int Sqp = nq * 128;
    Skp = nk * 128;
    wave = wave_;
    lane = lane_;
    const int g = lane >> 5;

    // Q fragments (B operand of S^T): query row qrow, bytes [64 hh + 32 g, +32)
    qrow = I * 128 + wave * 32 + (lane & 31);
    if constexpr (!QF) {
      const uint8_t* qp = q8 + ((int64_t)bh * Sqp + qrow) * D + 32 * g;
#pragma unroll
      for (int hh = 0; hh < D / 64; ++hh) {
        const v4i lo = *reinterpret_cast<const v4i*>(qp + 64 * hh);
        const v4i hi = *reinterpret_cast<const v4i*>(qp + 64 * hh + 16);
        qf[hh][0] = lo[0]; qf[hh][1] = lo[1]; qf[hh][2] = lo[2]; qf[hh][3] = lo[3];
        qf[hh][4] = hi[0]; qf[hh][5] = hi[1]; qf[hh][6] = hi[2]; qf[hh][7] = hi[3];
      }
      sqI = sq[(int64_t)bh * nq + I];
    }
    skh = sk + (int64_t)bh * nk;

    krs = __builtin_amdgcn_make_buffer_rsrc((void*)(k8 + (int64_t)bh * Skp * D), 0, Skp * D, 0x00020000);
    vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(v8t + (int64_t)bh * D * Skp), 0, D * Skp, 0x00020000);
    brs = krs;
    mrs = krs;
    if constexpr (HAS_BIAS)
      brs = __builtin_amdgcn_make_buffer_rsrc((void*)(key_bias + (int64_t)b * Sk), 0, Sk * 4, 0x00020000);
    if constexpr (HAS_MASK)
      mrs = __builtin_amdgcn_make_buffer_rsrc((void*)(key_mask + (int64_t)b * Sk), 0, Sk, 0x00020000);
    brow = HAS_BIAS ? key_bias + (int64_t)b * Sk : nullptr;
    mrow = HAS_MASK ? key_mask + (int64_t)b * Sk : nullptr;
    // Per-lane DMA offsets.  A 1 KB DMA instruction J fills LDS bytes [1024 J, +1024): lane
    // i writes 16 bytes at row 8J + i/8 (128-byte rows) or 16J + i/4 (64-byte rows),
    // physical chunk i%8 (i%4), which must hold logical chunk phys ^ lds_swz(row); for
    // 128-byte rows that depends on the parity of J, hence one offset per parity.
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
  }

  // The Q quantizer of this work item's 128-row block, fused: q~ = fp32(q) * c, sq =
  // max(max|q~|, 1e-12) / 448 over the block, codes e4m3(clamp(q~ / sq)) -- the arithmetic
  // of attn_quant_qk_kernel, so the scale and the fragments of rows < Sq are bit-identical
  // to its sq / q8.  red: 4 floats of LDS no DMA writes before the next attn_barrier.  Ends
  // with a workgroup barrier.
  template <int QDT>
  __device__ __forceinline__ void quant_q(const AttnQ16& qa, int Sq, int nq, float* red) {
    uint4 raw[D / 64][4];
    load_q16(qa, b, h, qrow, Sq, lane, raw);
    quant_q_raw<QDT>(raw, qa, nq, red);
  }

  // The 16-bit Q values this lane quantizes: row `row` of head (b_, h_), bytes
  // [64 hh + 32 g, +32) of its codes.  A row >= Sq reads row Sq - 1 (of the same 128-row
  // block): a copy of one of the block's rows leaves the block maximum as it is, and the
  // query of a row past Sq is computed but never stored (every statistic of the kernel is
  // per query), so its codes need no masking.  The loads stay unconditional and nothing
  // touches their registers before they are consumed, so no wait lands where they are
  // issued and no branch splits the count of loads in flight that later waits rely on.
  static __device__ __forceinline__ void load_q16(const AttnQ16& qa, int b_, int h_, int row, int Sq, int lane_,
                                                  uint4 (&raw)[D / 64][4]) {
    const int g = lane_ >> 5;
    const uint16_t* qp =
        qa.q + (int64_t)b_ * qa.sb + (int64_t)h_ * qa.sh + (int64_t)(row < Sq ? row : Sq - 1) * qa.ss + 32 * g;
#pragma unroll
    for (int hh = 0; hh < D / 64; ++hh)
#pragma unroll
      for (int u = 0; u < 4; ++u) raw[hh][u] = *reinterpret_cast<const uint4*>(qp + 64 * hh + 8 * u);
  }

  // First half of the Q quantizer: f = fp32(q) * c for this lane's 64 values and the wave's
  // max |f|.
  template <int QDT>
  static __device__ __forceinline__ float quant_q_scaled(const uint4 (&raw)[D / 64][4], float c,
                                                         float (&f)[D / 64][32]) {
    float amax = 0.0f;
#pragma unroll
    for (int hh = 0; hh < D / 64; ++hh)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint4 r = raw[hh][u];
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[hh][8 * u + 2 * i] = Elem<QDT>::lo(w[i]) * c;
          f[hh][8 * u + 2 * i + 1] = Elem<QDT>::hi(w[i]) * c;
          amax = fmaxf(amax, fabsf(f[hh][8 * u + 2 * i]));
          amax = fmaxf(amax, fabsf(f[hh][8 * u + 2 * i + 1]));
        }
      }
    return wave_max(amax);
  }

  // Second half: the block scale from the block maximum, the codes (Q fragments) and, when
  // qa.sq_out is set, the scale written out.
  __device__ __forceinline__ void quant_q_codes(const float (&f)[D / 64][32], float amax, const AttnQ16& qa, int nq) {
    const float sc = e4m3_scale(amax);
    const float r = __fdiv_rn(1.0f, sc);
#pragma unroll
    for (int hh = 0; hh < D / 64; ++hh)
#pragma unroll
      for (int k = 0; k < 8; ++k)
        qf[hh][k] = (int)cvt4_e4m3(clamp448(div_by_scale(f[hh][4 * k], sc, r)),
                                   clamp448(div_by_scale(f[hh][4 * k + 1], sc, r)),
                                   clamp448(div_by_scale(f[hh][4 * k + 2], sc, r)),
                                   clamp448(div_by_scale(f[hh][4 * k + 3], sc, r)));
    sqI = sc;
    if (qa.sq_out != nullptr && wave == 0 && lane == 0) qa.sq_out[(int64_t)bh * nq + I] = sc;
  }

  // The whole quantizer, the block maximum going through red and a workgroup barrier.
  template <int QDT>
  __device__ __forceinline__ void quant_q_raw(const uint4 (&raw)[D / 64][4], const AttnQ16& qa, int nq, float* red) {
    float f[D / 64][32];
    float amax = quant_q_scaled<QDT>(raw, qa.c, f);
    if (lane == 0) red[wave] = amax;
    attn_barrier();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    quant_q_codes(f, amax, qa, nq);
  }

  // Key tile (keys [kv0, kv0 + 128)) -> sK, rows permuted by key_of_row.
  __device__ __forceinline__ void dma_k(uint8_t* sK, int kv0) const {
    typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
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
  }

  // V^T tile (D rows x keys [kv0, kv0 + 128)) -> sV.
  __device__ __forceinline__ void dma_v(uint8_t* sV, int kv0) const {
    typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
#pragma unroll
    for (int j = 0; j < T::V_INSTR; ++j) {
      const int J = wave * T::V_INSTR + j;  // V^T rows [8J, 8J + 8)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, LDS_PTR(sV + J * 1024), 16, v_lane[j & 1], 8 * J * Skp + kv0, 0,
                                               0);
    }
  }

  // Mask / bias of keys [kv0, kv0 + 128) -> sAux (bias fp32 at 0, mask bytes at 1024).  Full
  // tiles use the DMA; the partial last tile loads element by element with a bounds check
  // (a 16-byte DMA chunk that straddles the end of a [B, Sk] row is range-checked as a
  // whole and would read back as zeros).
  __device__ __forceinline__ void dma_aux(uint8_t* sAux, int kv0, int Sk) const {
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
            b4[e] = key < Sk ? brow[key] : 0.0f;
          }
          *reinterpret_cast<v4f*>(sAux + 16 * lane) = b4;
        }
      }
    }
    if constexpr (HAS_MASK) {
      if (wave == 1) {
        if (!tail) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(mrs, LDS_PTR(sAux + 1024), 16, (uint32_t)(kv0 + (lane & 7) * 16),
                                                   0, 0, 0);
        } else if (lane < 8) {
          uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = kv0 + 16 * lane + e;
            const uint32_t byte = key < Sk ? (uint32_t)mrow[key] : 0u;
            w[e >> 2] |= byte << (8 * (e & 3));
          }
          *reinterpret_cast<v4i*>(sAux + 1024 + 16 * lane) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
      }
    }
  }
};

// Running state of a wave's 32 queries.  With the repair, the corrections go into the same
// accumulators: O and O_r (and the two parts of l) are scaled by the same factors and only
// their sum is used, so one set holds both (fp32 summation order is all that changes).
template <int D>
struct AttnState {
  static constexpr int NDT = D / 32;  // O^T row tiles
  v16f o[NDT];
  // Running sums of the P codes (and repair corrections) from the 16x16x128 row-sum
  // product: lane n < 16 holds query n's in register 0 and query n + 16's in register 1
  // (see AttnMfmaRun, x == NDT).
  v4f lacc;
  float m;  // lazy row max (log2 domain)
  // the code constants that depend on m (see attn_codes_w4): 7 - m and (48 - 8 m) 2^64
  float cst8, cstf;

  __device__ __forceinline__ void set_m(float m_new) {
    m = m_new;
    cst8 = 7.0f - m_new;
    cstf = (48.0f - 8.0f * m_new) * 0x1p64f;
  }

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) lacc[i] = 0.0f;
    set_m(kAttnNeg);
  }

  // O, l *= alpha (a moved lazy max)
  __device__ __forceinline__ void rescale(float alpha) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    // register 1 of lane n holds query n + 16's sum: it takes that query's alpha
    const float alpha16 = __shfl(alpha, ((int)(__lane_id() & 15)) + 16, 64);
    lacc[0] *= alpha;
    lacc[1] *= alpha16;
  }
};

// Lane offsets of the 16-byte LDS chunks a lane reads for its MFMA A fragments.  Row
// 32x + r of a swizzled tile has the same swizzle as row r (lds_swz depends on row / 2 or
// row / 4 modulo 8 / 4), so the subtile (t) and channel-tile (dt) offsets are immediates.
template <int D>
struct AttnFragOfs {
  int k[D / 64][2];  // K tile: half hh, chunk 4 hh + 2 g + e
  int v[2][2];       // V^T tile: key half kh, chunk 4 kh + 2 g + e
  // A operand of the 16x16x128 row-sum product over one 64-key half of P.  As its B
  // operand, the PV fragment of lane l holds 32 codes of query l % 32; the product reads
  // lane n + 16 j as column n, k range [32 j, +32), i.e. query n for j = 0, 2 and query
  // n + 16 for j = 1, 3.  Row 0 of A is 1.0 (e4m3 0x38) on k groups 0 and 2, row 1 on
  // groups 1 and 3, other rows 0: output row 0 is query n's sum, row 1 query n + 16's.
  v8i rowsum_sel;
  __device__ __forceinline__ explicit AttnFragOfs(int lane) {
    const int r = lane & 31, g = lane >> 5;
    {
      const int row = lane & 15, j = lane >> 4;
      const bool one = (row == 0 && (j & 1) == 0) || (row == 1 && (j & 1) == 1);
      const int w = one ? 0x38383838 : 0;
      rowsum_sel = v8i{w, w, w, w, w, w, w, w};
    }
#pragma unroll
    for (int hh = 0; hh < D / 64; ++hh)
#pragma unroll
      for (int e = 0; e < 2; ++e) k[hh][e] = r * D + (((4 * hh + 2 * g + e) ^ lds_swz<D>(r)) << 4);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 2; ++e) v[kh][e] = r * 128 + (((4 * kh + 2 * g + e) ^ lds_swz<128>(r)) << 4);
  }
};

__device__ __forceinline__ v8i lds_pair(const uint8_t* base, int o0, int o1) {
  const v4i lo = *reinterpret_cast<const v4i*>(base + o0);
  const v4i hi = *reinterpret_cast<const v4i*>(base + o1);
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// Four fp32 values divided by 16 -> four e4m3fn bytes (RNE), packed little-endian: the
// scaled conversion divides by its scale before rounding, so these are the codes of a / 16 ..
// d / 16 exactly.
__device__ __forceinline__ int cvt4_e4m3_div16(float a, float b, float c, float d) {
  typedef short v2s __attribute__((ext_vector_type(2)));
  const v2s lo = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(v2s{0, 0}, a, b, 16.0f, false);
  const v2s hi = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(lo, c, d, 16.0f, true);
  return __builtin_bit_cast(int, hi);
}

// E8M0 block scale of the repair operands: the two e4m3 parts of 8 delta are multiplied
// by 2^-3 inside the product (127 = 1.0).
constexpr int kRepairScaleE8M0 = 124;

// B operands of the PV products of one tile: the P codes and, with the repair, the two
// e4m3 parts hi + lo = 8 delta of the corrections (zero where no correction applies).
template <bool REP>
struct AttnPB {
  v8i p[2];
  v8i hi[REP ? 2 : 1];
  v8i lo[REP ? 2 : 1];
};

// Per-tile constants of the code arithmetic (see attn_codes_w4).
struct AttnCodeK {
  float c1, cst8, c8f, cstf;
  uint32_t rep_add;  // the repair threshold as a byte addend (attn_repair_addend)
  // cst8 = 7 - m_new and cstf = (48 - 8 m_new) 2^64 come with the row max (AttnState)
  template <bool HAS_BIAS>
  __device__ __forceinline__ static AttnCodeK make(float sq, float skj, float cst8, float cstf, uint32_t rep_add) {
    AttnCodeK k;
    k.cst8 = cst8;
    // sq sk, exactly an eighth of the rounded (8 sq) sk
    k.c1 = HAS_BIAS ? 1.0f : sq * skj;
    k.c8f = (k.c1 * 8.0f) * 0x1p64f;
    k.cstf = cstf;
    k.rep_add = rep_add;
    return k;
  }
};

// The repair threshold (kernels/fp8_attention.py:290, P >= tau) on the codes themselves: P is
// the value of its e4m3 code, and code values grow with the code, so P >= tau exactly when
// code >= T, T the smallest code whose value is >= tau (127 when none is: codes stay <= 120).
// Added to a word of four codes (each <= 0x7e), (0x80 - T) per byte sets a byte's top bit
// exactly when its code is >= T, with no carry between bytes.
static inline uint32_t attn_repair_addend(float tau) {
  int T = 127;
  for (int c = 0; c < 127; ++c) {
    const int e = c >> 3, m = c & 7;
    const float v = e == 0 ? m * 0x1p-9f : ldexpf(1.0f + m * 0.125f, e - 7);
    if (v >= tau) {
      T = c;
      break;
    }
  }
  return (uint32_t)(0x80 - T) * 0x01010101u;
}

// The exp2-free P codes of scores 4 w4 .. 4 w4 + 3 of score subtile t: word 4 (t & 1) + w4
// of the PV B operand of key half t >> 1.
//
// code = bits < 8 ? 0 : rint(bits), bits = 8 S + 56 - 8 m_new.  bits never exceeds
// 8 * 8 + 56 = 120 (the lazy max keeps S <= m + 8), so the reference's clamp to [0, 126] is
// inactive.  Three FMAs per score, all at the full FMA rate, on b = bits / 8 (exactly: an
// eighth of every term, so b = RN(bits) / 8):
//   b    = fma(dot, c1, cst8)                                (c1 = sq sk, cst8 = 7 - m)
//   keep = clamp01(fma(dot, 8 c1 2^64, (48 - 8 m) 2^64))     (1 when bits >= 8, else 0)
//   t    = fma(b, keep, 1.5 * 2^20)
// keep uses the FMA's free output clamp: the argument is (exact bits - 8) * 2^64, so keep
// is 0 exactly when bits < 8 (and for invalid keys, whose product overflows to -inf) and
// 1 once bits exceeds 8 by 2^-64.  Adding 1.5 * 2^20, whose ulp is 2^-3, rounds b to a
// multiple of 1/8 with the FMA's round-to-nearest-even, i.e. rounds bits to an integer, and
// leaves rint(bits) in the low mantissa bits of t (0 when keep is 0), so v_perm_b32 packs the
// low bytes of four t's into one dword of codes.
//
// Repair (REP, kernels/fp8_attention.py:288-292): delta = exp2(S - m) - P where P >= tau,
// else 0.  exp2(b) = exp2(S - m + 7) = 128 exp2(S - m); P is the decoded code.  delta is
// bounded by about 11% of exp2(S - m) <= 2^8 (the code's relative error: Mitchell's 6.1% and
// the rounding of bits), so |8 delta| < 448 and 8 delta splits into e4m3 parts
// hi = e4m3(8 delta), lo = e4m3(8 delta - hi) (the remainder is exact in fp32), which the
// PV products multiply with V at the block scale 2^-3.  The conversions take 128 delta and
// divide it by 16 themselves (v_cvt_scalef32_*: the same codes as plain conversions of
// 8 delta, and decoded values 16 times theirs).  hi + lo holds 8 delta to about 8
// significant bits (exactly its bf16 rounding's precision for |8 delta| >= 2^-2; below that
// lo's e4m3 grid, 2^-9, bounds the error), where the reference rounds delta to bf16.
template <bool REP>
__device__ __forceinline__ void attn_codes_w4(const v16f& st, const AttnCodeK& k, int t, int w4, AttnPB<REP>& pb) {
  {
    uint32_t tb[4];
    float b8[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = st[4 * w4 + e];
      b8[e] = __builtin_fmaf(x, k.c1, k.cst8);
      const float keep = __builtin_amdgcn_fmed3f(__builtin_fmaf(x, k.c8f, k.cstf), 0.0f, 1.0f);
      tb[e] = __float_as_uint(__builtin_fmaf(b8[e], keep, 1572864.0f));
    }
    // bytes [t0, t1, 0, 0] | [0, 0, t2, t3]
    const uint32_t word = __builtin_amdgcn_perm(tb[1], tb[0], 0x0c0c0400u) |
                          __builtin_amdgcn_perm(tb[3], tb[2], 0x04000c0cu);
    // An empty use keeps the codes here instead of letting them sink to their consumer
    // (the PV products): a reordered tile would hold the scores and the codes live together.
    asm volatile("" ::"v"(word));
    pb.p[t >> 1][4 * (t & 1) + w4] = (int)word;
    if constexpr (REP) {
      const v2f p01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
      const v2f p23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true);
      const float papx[4] = {p01[0], p01[1], p23[0], p23[1]};
      float d[4];  // 128 delta
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // invalid keys: b ~ -1e29, exp2 -> 0 and the code is 0, so delta = 0
        d[e] = __builtin_fmaf(papx[e], -128.0f, __builtin_amdgcn_exp2f(b8[e]));
      }
      const int hi = cvt4_e4m3_div16(d[0], d[1], d[2], d[3]);
      const v2f h01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 16.0f, false);
      const v2f h23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 16.0f, true);
      const int lo = cvt4_e4m3_div16(d[0] - h01[0], d[1] - h01[1], d[2] - h23[0], d[3] - h23[1]);
      // codes below the threshold take no correction: their hi and lo bytes are cleared.
      // Byte k of the mask is the top bit of byte k of word + rep_add, spread over the byte
      // (v_perm's sign-replicating selectors: bytes 1, 3 of the low source and 5, 7 of the
      // high one, which holds the flags shifted up by a byte)
      const uint32_t flag = word + k.rep_add;
      const int mask = (int)__builtin_amdgcn_perm(flag << 8, flag, 0x090b080au);
      pb.hi[t >> 1][4 * (t & 1) + w4] = hi & mask;
      pb.lo[t >> 1][4 * (t & 1) + w4] = lo & mask;
    }
  }
}

// The codes of score subtile t.
template <bool REP>
__device__ __forceinline__ void attn_codes_sub(const v16f& st, const AttnCodeK& k, int t, AttnPB<REP>& pb) {
#pragma unroll
  for (int w4 = 0; w4 < 4; ++w4) attn_codes_w4<REP>(st, k, t, w4, pb);
}

// A run of matrix-core products with their A fragments fetched from LDS AHEAD products
// ahead (AHEAD + 1 fragments in flight), so the products issue back to back instead of
// each waiting for its own LDS read.  The run is the PV products of key halves
// [KH0, KH1) of one tile (per half: O^T tile x for x < D/32, then the row-sum product at
// x == D/32; with REP each fragment also multiplies the two repair parts) followed by the
// QK^T products of score subtiles [U0, U1) of another (per subtile: the D/64 channel
// halves hh).
template <int D, int KH0, int KH1, int U0, int U1, int AHEAD = 3>
struct AttnMfmaRun {
  static constexpr int RING = AHEAD + 1;
  static constexpr int NDT = D / 32, QKM = D / 64;
  static constexpr int NPV = (KH1 - KH0) * (NDT + 1), NQK = (U1 - U0) * QKM, N = NPV + NQK;

  template <int K>
  __device__ static __forceinline__ v8i frag(const uint8_t* sV, const uint8_t* sK, const AttnFragOfs<D>& fo) {
    if constexpr (K < NPV) {
      constexpr int kh = KH0 + K / (NDT + 1), x = K % (NDT + 1);
      if constexpr (x == NDT)
        return fo.rowsum_sel;
      else
        return lds_pair(sV + x * 32 * 128, fo.v[kh][0], fo.v[kh][1]);
    } else {
      constexpr int u = U0 + (K - NPV) / QKM, hh = (K - NPV) % QKM;
      return lds_pair(sK + u * 32 * D, fo.k[hh][0], fo.k[hh][1]);
    }
  }

  template <int K, bool REP>
  __device__ static __forceinline__ void exec(const v8i& fr, const AttnPB<REP>& pb, const v8i (&qf)[D / 64],
                                              v16f (&s)[4], AttnState<D>& st) {
    if constexpr (K < NPV) {
      constexpr int kh = KH0 + K / (NDT + 1), x = K % (NDT + 1);
      if constexpr (x == NDT) {
        st.lacc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fr, pb.p[kh], st.lacc, 0, 0, 0, 0, 0, 0);
        if constexpr (REP) {
          st.lacc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fr, pb.hi[kh], st.lacc, 0, 0, 0, 127, 0,
                                                                     kRepairScaleE8M0);
          st.lacc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fr, pb.lo[kh], st.lacc, 0, 0, 0, 127, 0,
                                                                     kRepairScaleE8M0);
        }
      } else {
        st.o[x] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr, pb.p[kh], st.o[x], 0, 0, 0, 0, 0, 0);
        if constexpr (REP) {
          st.o[x] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr, pb.hi[kh], st.o[x], 0, 0, 0, 127, 0,
                                                                    kRepairScaleE8M0);
          st.o[x] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr, pb.lo[kh], st.o[x], 0, 0, 0, 127, 0,
                                                                    kRepairScaleE8M0);
        }
      }
    } else {
      constexpr int u = U0 + (K - NPV) / QKM, hh = (K - NPV) % QKM;
      if constexpr (hh == 0) {
        v16f z;
#pragma unroll
        for (int i = 0; i < 16; ++i) z[i] = 0.0f;
        s[u] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr, qf[0], z, 0, 0, 0, 0, 0, 0);
      } else {
        s[u] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr, qf[hh], s[u], 0, 0, 0, 0, 0, 0);
      }
    }
  }

  template <int K, bool REP>
  __device__ static __forceinline__ void seq(v8i (&fr)[RING], const uint8_t* sV, const uint8_t* sK,
                                             const AttnFragOfs<D>& fo, const AttnPB<REP>& pb,
                                             const v8i (&qf)[D / 64], v16f (&s)[4], AttnState<D>& st) {
    if constexpr (K < N) {
      if constexpr (K + AHEAD < N) fr[(K + AHEAD) % RING] = frag<K + AHEAD>(sV, sK, fo);
      exec<K, REP>(fr[K % RING], pb, qf, s, st);
      // keep program order: a reordered run would hold the scores and the PV fragments
      // live together
      __builtin_amdgcn_sched_barrier(0);
      seq<K + 1, REP>(fr, sV, sK, fo, pb, qf, s, st);
    }
  }

  // the first AHEAD fragments of the run
  template <int K>
  __device__ static __forceinline__ void prime(v8i (&fr)[RING], const uint8_t* sV, const uint8_t* sK,
                                               const AttnFragOfs<D>& fo) {
    if constexpr (K < AHEAD && K < N) {
      fr[K] = frag<K>(sV, sK, fo);
      prime<K + 1>(fr, sV, sK, fo);
    }
  }

  template <bool REP>
  __device__ static __forceinline__ void run(const uint8_t* sV, const uint8_t* sK, const AttnFragOfs<D>& fo,
                                             const AttnPB<REP>& pb, const v8i (&qf)[D / 64], v16f (&s)[4],
                                             AttnState<D>& st) {
    v8i fr[RING];
    prime<0>(fr, sV, sK, fo);
    seq<0, REP>(fr, sV, sK, fo, pb, qf, s, st);
  }
};

// Score given to invalid keys: finite and so negative that it loses every row max and
// flushes to code 0.  The flush test multiplies it by c8 = 8 sq sk (or 8 with a bias), so
// it is chosen to make that product -1e30 (finite: no inf * 0 = NaN downstream); for
// c8 < 1e-8 it is -1e38 and the product is smaller still.
template <bool HAS_BIAS>
__device__ __forceinline__ float attn_invalid_score(float sq, float skj) {
  if constexpr (HAS_BIAS) return -1.25e29f;
  return -1.0e30f / fmaxf((8.0f * sq) * skj, 1.0e-8f);
}

// Whether tile [kv0, kv0 + 128) has any invalid key (wave-uniform).  A bias applies to
// every score; a key mask only matters when one of the tile's 128 mask bytes (LDS, at
// sAux + 1024) is zero: lanes 0-31 test one dword each for a zero byte.
template <bool HAS_MASK, bool HAS_BIAS>
__device__ __forceinline__ bool attn_tile_needs_mask(const uint8_t* sAux, int kv0, int Sk, int lane) {
  if (HAS_BIAS || kv0 + 128 > Sk) return true;
  if constexpr (!HAS_MASK) {
    return false;
  } else {
    const uint32_t w = lane < 32 ? *reinterpret_cast<const uint32_t*>(sAux + 1024 + 4 * lane) : 0x01010101u;
    const bool has_zero_byte = ((w - 0x01010101u) & ~w & 0x80808080u) != 0u;
    return __builtin_amdgcn_ballot_w64(has_zero_byte) != 0;
  }
}

// Every key of the tile masked out (a key mask and no bias; keys past Sk read as masked):
// its scores would all take the masked value, which moves no row max, and its codes would
// all be 0, adding exact zeros to O and l -- so the kernels skip its softmax and PV
// products.
template <bool HAS_MASK, bool HAS_BIAS>
__device__ __forceinline__ bool attn_tile_all_masked(const uint8_t* sAux, int lane) {
  if constexpr (!HAS_MASK || HAS_BIAS) {
    return false;
  } else {
    const uint32_t w = lane < 32 ? *reinterpret_cast<const uint32_t*>(sAux + 1024 + 4 * lane) : 0u;
    return __builtin_amdgcn_ballot_w64(w != 0u) == 0;
  }
}

// S = (dot * sq) * sk + bias * log2(e) with every operation rounded on its own, as the
// reference's statements are (kernels/fp8_attention.py:253, 259).  Contraction is off here:
// an FMA that one kernel forms and another does not would move S by an ulp, which decides
// ties of the code's rounding, so that kernels of the same arithmetic would not give the
// same bits.
__device__ __forceinline__ float attn_bias_score(float dot, float sq, float skj, float bias) {
#pragma clang fp contract(off)
  return (dot * sq) * skj + bias * 1.4426950408889634f;
}

// Invalid keys (past Sk, masked, bias <= -1e8) get attn_invalid_score; with a bias S is
// formed explicitly as (dot * sq) * sk + bias * log2 e.
// Score subtiles [T0, T0 + NT).
template <bool HAS_MASK, bool HAS_BIAS, int T0 = 0, int NT = 4>
__device__ __forceinline__ void attn_mask_scores(v16f (&s)[4], const uint8_t* sAux, int kv0, int Sk, float sq,
                                                 float skj, int lane) {
  const int g = lane >> 5;
  const float vinv = attn_invalid_score<HAS_BIAS>(sq, skj);
#pragma unroll
  for (int t = T0; t < T0 + NT; ++t) {
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
        v = attn_bias_score(v, sq, skj, bias[i]);
      }
      if constexpr (HAS_MASK) ok = ok && (((mbytes[i >> 2] >> (8 * (i & 3))) & 0xffu) != 0u);
      s[t][i] = ok ? v : vinv;
    }
  }
}

// Row max over score subtiles [T0, T0 + NT) (exactly the reference's fp32 S max over
// those keys: x -> (x * sq) * sk is monotonic), floored at -1e9.  Four independent v_max3
// chains, so that the VALU need not wait on each result.
template <bool HAS_BIAS, int T0 = 0, int NT = 4>
__device__ __forceinline__ float attn_part_max(const v16f (&s)[4], float sq, float skj) {
  float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int t = T0; t < T0 + NT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) m4[i & 3] = fmaxf(m4[i & 3], s[t][i]);
  float mx = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
  {
    // partner lane^32 through v_permlane32_swap (two copies: each half receives the other).
    // Both values come from arithmetic, so neither is a signaling NaN, and for those a plain
    // v_max_f32 is fmaxf (a quiet NaN yields the other operand).  Written out, because the
    // compiler would first canonicalize both operands, a quieting only signaling NaNs need.
    const uint32_t u = __float_as_uint(mx);
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    asm("v_max_f32 %0, %1, %2" : "=v"(mx) : "v"(__uint_as_float(sw[0])), "v"(__uint_as_float(sw[1])));
  }
  return fmaxf(HAS_BIAS ? mx : (mx * sq) * skj, kAttnNeg);
}

// The lazy-max decision (kernels/fp8_attention.py:264): the row max moves to the tile's
// maximum rmax only when that exceeds it by more than 8, or while it is still -1e9.  The
// second test changes nothing here: rmax >= -1e9 (attn_part_max clamps it) and -1e9 + 8
// rounds to -1e9 in fp32 (its ulp is 64), so with m_old = -1e9 either rmax > m_old + 8 or
// rmax = -1e9 = m_old, and both branches give rmax.  Returns whether the max moves.
__device__ __forceinline__ bool attn_max_moves(float rmax, float m_old) { return rmax > m_old + 8.0f; }

// One tile's row max and lazy-max decision, the rescale of O and l when the max moves
// (rescale = false: they are still zero, and scaling them would change no bit), and the
// tile's codes.  Rows whose max stays take alpha = 1 in a rescale, which changes no bit.
template <bool HAS_BIAS, bool REP, int D>
__device__ __forceinline__ void attn_softmax_tile(const v16f (&s)[4], float sq, float skj, uint32_t rep_add,
                                                  bool rescale,
                                                  AttnState<D>& st, AttnPB<REP>& pb) {
  const float rmax = attn_part_max<HAS_BIAS>(s, sq, skj);
  const bool moves = attn_max_moves(rmax, st.m);
  if (__builtin_amdgcn_ballot_w64(moves)) {
    const float m_new = moves ? rmax : st.m;
    if (rescale) st.rescale(__builtin_amdgcn_exp2f(st.m - m_new));
    st.set_m(m_new);
  }
  const AttnCodeK k = AttnCodeK::make<HAS_BIAS>(sq, skj, st.cst8, st.cstf, rep_add);
#pragma unroll
  for (int t = 0; t < 4; ++t) attn_codes_sub<REP>(s[t], k, t, pb);
}

// The channel scales sv of head bh that this lane's output channels take (see attn_store).
// They are loaded, and every load in flight waited for, before the first output store:
// loads and stores retire in order, so a load still in flight behind a store would make
// any later wait for it wait for the store as well.
template <int D>
struct AttnSv {
  v4f r[D / 32][4];
  __device__ __forceinline__ void load(const float* sv, int bh, int lane) {
    const float* svh = sv + (int64_t)bh * D + 4 * (lane >> 5);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) r[dt][q4] = *reinterpret_cast<const v4f*>(svh + 32 * dt + 8 * q4);
    wait_vm0();
  }
  // from a copy of the head's D scales in LDS
  __device__ __forceinline__ void load_lds(const float* svl, int lane) {
    const float* s = svl + 4 * (lane >> 5);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) r[dt][q4] = *reinterpret_cast<const v4f*>(s + 32 * dt + 8 * q4);
  }
};

// O = (O + O_r) * sv / max(l, 1e-12) -> out (bf16 / fp16 through its strides; O_r is inside
// O).  The lane holds query qrow, channels 32 dt + 8 (i/4) + 4 g + i%4.
template <int D, int ODT>
__device__ __forceinline__ void attn_store(const AttnState<D>& st, const AttnSv<D>& svr, int b, int h, int qrow,
                                           int lane, void* out, int64_t os_b, int64_t os_h, int64_t os_s,
                                           int64_t os_d) {
  constexpr int NDT = D / 32;
  const int g = lane >> 5;
  // row sum of this lane's query q = lane % 32: register q / 16 of lane q % 16
  const int q = lane & 31;
  const float l0 = __shfl(st.lacc[0], q & 15, 64), l1 = __shfl(st.lacc[1], q & 15, 64);
  const float l = q < 16 ? l0 : l1;
  const float den = fmaxf(l, 1.0e-12f);
  // (acc * sv) / den correctly rounded from one reciprocal per row (div_by_scale: the
  // quotients are O's values and den lies in [1e-12, ~1e7], so nothing over- or underflows)
  const float rden = __fdiv_rn(1.0f, den);
  char* obase = static_cast<char*>(out) + ((int64_t)b * os_b + (int64_t)h * os_h + (int64_t)qrow * os_s) * 2;
  // channels d0 .. d0 + 3 of chunk (dt, q4) as two packed 16-bit pairs
  uint32_t ob[NDT][4][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = div_by_scale(st.o[dt][4 * q4 + e] * svr.r[dt][q4][e], den, rden);
      ob[dt][q4][0] = cvt_pk_16<ODT>(v[0], v[1]);
      ob[dt][q4][1] = cvt_pk_16<ODT>(v[2], v[3]);
    }
  uint16_t* orow = reinterpret_cast<uint16_t*>(obase);
  if (os_d == 1) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * q4 + 4 * g) = make_uint2(ob[dt][q4][0], ob[dt][q4][1]);
  } else {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint16_t* dst = orow + (int64_t)(32 * dt + 8 * q4 + 4 * g) * os_d;
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(int64_t)e * os_d] = (uint16_t)(ob[dt][q4][e >> 1] >> (16 * (e & 1)));
      }
  }
}

// attn_store for a wave's whole block of 32 query rows, in two steps.  attn_stage_rows goes
// through a 2 KB LDS region of the wave's own (stage): per 32 channels, the lanes write their
// 8-byte pairs of packed values to the rows they hold, then read back 16 bytes each, so that
// attn_write_rows' store instructions write 16 whole 64-byte row segments (non-temporal)
// instead of 32 rows x 16 bytes.  16-byte chunks are XOR-swizzled by row / 4, so the writes
// hit each bank at most twice and the reads not at all more than the 16-byte width needs.
// The staged rows are held in registers between the two steps.  wrow0: the block's first
// row; row_bytes / col_bytes: the row and channel strides in bytes; vec: col_bytes == 2 and
// wrow0, row_bytes 16-byte aligned (one 16-byte store per chunk; otherwise eight 2-byte
// stores).  Rows at or past nvalid are not stored.  Same values as attn_store.
__device__ __forceinline__ int attn_stage_chunk(int row, int c) { return (row * 64) + ((c ^ ((row >> 2) & 3)) << 4); }

// The staged rows of a wave, 16 bytes per lane and 32-channel slice for rows lane / 4 and
// lane / 4 + 16.
template <int D>
struct AttnStaged {
  v4i a[D / 32], b[D / 32];
};

template <int D, int ODT>
__device__ __forceinline__ void attn_stage_rows(const AttnState<D>& st, const AttnSv<D>& svr, int lane,
                                                uint8_t* stage, AttnStaged<D>& r) {
  constexpr int NDT = D / 32;
  const int g = lane >> 5;
  const int q = lane & 31;
  const float l0 = __shfl(st.lacc[0], q & 15, 64), l1 = __shfl(st.lacc[1], q & 15, 64);
  const float l = q < 16 ? l0 : l1;
  const float den = fmaxf(l, 1.0e-12f);
  const float rden = __fdiv_rn(1.0f, den);
  // read-back: lane L holds row L / 4 (+ 16), chunk L % 4 of the 64-byte row segment
  const int rr = lane >> 2, c = lane & 3;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = div_by_scale(st.o[dt][4 * q4 + e] * svr.r[dt][q4][e], den, rden);
      *reinterpret_cast<uint2*>(stage + attn_stage_chunk(q, q4) + 8 * g) =
          make_uint2(cvt_pk_16<ODT>(v[0], v[1]), cvt_pk_16<ODT>(v[2], v[3]));
    }
    r.a[dt] = *reinterpret_cast<const v4i*>(stage + attn_stage_chunk(rr, c));
    r.b[dt] = *reinterpret_cast<const v4i*>(stage + attn_stage_chunk(rr + 16, c));
  }
}

template <int D>
__device__ __forceinline__ void attn_write_rows(const AttnStaged<D>& r, char* wrow0, int64_t row_bytes,
                                                int64_t col_bytes, bool vec, int nvalid, int lane) {
  constexpr int NDT = D / 32;
  const int rr = lane >> 2, c = lane & 3;
  char* const dst0 = wrow0 + (int64_t)rr * row_bytes + 8 * c * col_bytes;
  char* const dst1 = dst0 + 16 * row_bytes;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    if (vec) {
      // non-temporal: the kernel never reads its output back, and the L2 keeps Q and K/V
      if (rr < nvalid) __builtin_nontemporal_store(r.a[dt], reinterpret_cast<v4i*>(dst0 + 64 * dt));
      if (rr + 16 < nvalid) __builtin_nontemporal_store(r.b[dt], reinterpret_cast<v4i*>(dst1 + 64 * dt));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t o = (32 * dt + e) * col_bytes;
        if (rr < nvalid) *reinterpret_cast<uint16_t*>(dst0 + o) = (uint16_t)(r.a[dt][e >> 1] >> (16 * (e & 1)));
        if (rr + 16 < nvalid)
          *reinterpret_cast<uint16_t*>(dst1 + o) = (uint16_t)(r.b[dt][e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// One tile at a time: per KV tile, S = QK^T, codes (and the repair parts), PV.  Two waves
// per SIMD (256 registers each), so one wave's softmax overlaps the other's products.
// ---------------------------------------------------------------------------------------

// QF: Q arrives as 16-bit values of the output's dtype (qa) and each workgroup quantizes
// its own 128-row block while its first KV tile is in flight; q8 / sq are then unused.
template <int D, bool HAS_MASK, bool HAS_BIAS, bool DO_REPAIR, int ODT, bool QF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void attn_fwd_kernel(const uint8_t* __restrict__ q8, const uint8_t* __restrict__ k8, const uint8_t* __restrict__ v8t,
                     const float* __restrict__ sq, const float* __restrict__ sk, const float* __restrict__ sv,
                     const uint8_t* __restrict__ key_mask, const float* __restrict__ key_bias, uint32_t rep_add,
                     void* __restrict__ out, int64_t os_b, int64_t os_h, int64_t os_s, int64_t os_d, int H, int Sq,
                     int Sk, int nq, AttnQ16 qa) {
  typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * T::BUF];
  AttnCtx<D, HAS_MASK, HAS_BIAS, QF> cx(q8, k8, v8t, sq, sk, key_mask, key_bias, H, Sk, nq,
                                        xcd_linear_id(blockIdx.x, gridDim.x),
                                        __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), threadIdx.x & 63);
  const int nk = cx.nk, lane = cx.lane;
  const AttnFragOfs<D> fo(lane);

  AttnState<D> st;
  st.init();

  const int j0 = (int)(((int64_t)cx.I * nk) / nq);
  cx.dma_k(smem, j0 * 128);
  cx.dma_v(smem + T::KB, j0 * 128);
  cx.dma_aux(smem + T::KB + T::VB, j0 * 128, Sk);
  // The block maximum goes through the second buffer, which the first DMA into it (after
  // the loop's first barrier) cannot reach before every wave has read it.
  if constexpr (QF) cx.template quant_q<ODT>(qa, Sq, nq, reinterpret_cast<float*>(smem + T::BUF));
  int j = j0;
  // Tile i uses buffer i & 1.  The loop takes the tiles in pairs so that each buffer's
  // address is a constant: the LDS fragment reads then carry it in their immediate offset
  // instead of adding it to every lane offset on every tile.
  auto tile = [&](auto par, int i) {
    constexpr int PAR = decltype(par)::value;
    // Tile i is the only DMA in flight; after the barrier every wave has finished tile
    // i-1, so its buffer can take tile i+1 while tile i is computed.
    wait_vm0();
    attn_barrier();
    const int jn = j + 1 == nk ? 0 : j + 1;
    if (i + 1 < nk) {
      uint8_t* nb = smem + (1 - PAR) * T::BUF;
      cx.dma_k(nb, jn * 128);
      cx.dma_v(nb + T::KB, jn * 128);
      cx.dma_aux(nb + T::KB + T::VB, jn * 128, Sk);
    }
    const uint8_t* buf = smem + PAR * T::BUF;
    const float skj = cx.skh[j];
    const int kv0 = j * 128;
    v16f s[4];
    AttnPB<DO_REPAIR> pb;
    AttnMfmaRun<D, 0, 0, 0, 4>::run(buf + T::KB, buf, fo, pb, cx.qf, s, st);
    if (attn_tile_needs_mask<HAS_MASK, HAS_BIAS>(buf + T::KB + T::VB, kv0, Sk, lane)) {
      // (tested here, where only tiles with a masked key pay for it)
      if (attn_tile_all_masked<HAS_MASK, HAS_BIAS>(buf + T::KB + T::VB, lane)) {
        j = jn;
        return;
      }
      attn_mask_scores<HAS_MASK, HAS_BIAS>(s, buf + T::KB + T::VB, kv0, Sk, cx.sqI, skj, lane);
    }
    attn_softmax_tile<HAS_BIAS>(s, cx.sqI, skj, rep_add, true, st, pb);
    AttnMfmaRun<D, 0, 2, 0, 0>::run(buf + T::KB, buf, fo, pb, cx.qf, s, st);
    j = jn;
  };
  for (int i = 0; i < nk; i += 2) {
    tile(std::integral_constant<int, 0>{}, i);
    if (i + 1 < nk) tile(std::integral_constant<int, 1>{}, i + 1);
  }
  AttnSv<D> svr;
  svr.load(sv, cx.bh, lane);
  if (cx.qrow >= Sq) return;
  attn_store<D, ODT>(st, svr, cx.b, cx.h, cx.qrow, lane, out, os_b, os_h, os_s, os_d);
}

// ---------------------------------------------------------------------------------------
// Short key sequences (all KV tiles of a head fit in LDS: Sk <= 512 at D = 128, <= 1024 at
// D = 64).  One persistent workgroup of 8 waves per CU walks a contiguous range of (head,
// Q tile) work items; the head's K, V^T (and mask / bias) tiles are copied into LDS once per
// head, and the two 4-wave groups take the range's Q tiles in pairs.  Per Q tile the
// arithmetic and the KV visit order are those of attn_fwd_kernel, so the output is the same
// bit for bit; what goes away is the per-tile copy and barrier and the per-workgroup
// start-up, which dominate when a Q tile has only a few KV tiles.  QF: Q arrives as 16-bit
// values and each group quantizes its own 128-row block (quant_q_raw); the block maximum
// goes through LDS among the group's 4 waves (AttnGroupX), one round per pair of tiles that
// every wave of the group takes part in (the loop over pairs is uniform across the
// workgroup), so the two groups run independently between head changes.  No repair path:
// the launcher uses attn_fwd_kernel for it.
// ---------------------------------------------------------------------------------------
template <int D>
struct AttnResident {
  static constexpr int NKMAX = D == 128 ? 4 : 8;  // KV tiles held in LDS
};

template <int D, bool HAS_MASK, bool HAS_BIAS, int ODT, bool QF>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void attn_fwd_resident_kernel(const uint8_t* __restrict__ q8, const uint8_t* __restrict__ k8,
                              const uint8_t* __restrict__ v8t, const float* __restrict__ sq,
                              const float* __restrict__ sk, const float* __restrict__ sv,
                              const uint8_t* __restrict__ key_mask, const float* __restrict__ key_bias,
                              void* __restrict__ out, int64_t os_b, int64_t os_h, int64_t os_s, int64_t os_d, int H,
                              int Sq, int Sk, int nq, int total, AttnQ16 qa) {
  typedef AttnTile<D, HAS_MASK || HAS_BIAS> T;
  constexpr int NKMAX = AttnResident<D>::NKMAX;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NKMAX * T::BUF];
  // QF: the block-maximum exchange of each group, one round per pair of tiles
  __shared__ AttnGroupX qgx[QF ? 2 : 1];
  // 2 KB per wave for the output stores (attn_stage_rows), where LDS has room for it
  constexpr bool STAGE = NKMAX * T::BUF + 8 * 2048 + D * 4 + 2 * (int)sizeof(AttnGroupX) <= 160 * 1024;
  __shared__ __attribute__((aligned(16))) uint8_t ostage[STAGE ? 8 * 2048 : 16];
  // whole 16-byte chunks of unit-stride rows
  const bool ovec = os_d == 1 && ((reinterpret_cast<uintptr_t>(out) | (uintptr_t)(os_b * 2) |
                                   (uintptr_t)(os_h * 2) | (uintptr_t)(os_s * 2)) & 15u) == 0;
  __shared__ __attribute__((aligned(16))) float svl[D];  // the loaded head's channel scales sv
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wq = wave & 3, lane = threadIdx.x & 63;
  const int nk = (Sk + 127) / 128;
  const AttnFragOfs<D> fo(lane);
  // XCD-contiguous ranges: the workgroups that share a head's K/V copies mostly sit on one
  // XCD, whose L2 then fetches them once
  const int L = xcd_linear_id(blockIdx.x, gridDim.x);
  const int ta = (int)(((int64_t)L * total) / gridDim.x);
  const int tb = (int)(((int64_t)(L + 1) * total) / gridDim.x);
  // Work item of this wave's group in the pair that starts at tile p: active when that
  // tile exists (p + grp < end of p's head segment), else a stand-in id.
  auto pair_item = [&](int p, bool& active) {
    const int seg_end = min(tb, (p / nq + 1) * nq);
    active = p + grp < seg_end;
    return active ? p + grp : p;
  };
  // The next tile's Q fragments and scale are fetched before the current tile's output
  // stores: loads and stores retire in order, so a load issued after the stores would wait
  // for them to reach memory.
  // QF: the next tile's 16-bit Q rows instead (zeros past Sq).
  v8i qnext[D / 64];
  float sqnext = 0.0f;
  uint4 rawnext[QF ? D / 64 : 1][4];
  // QF: the next item's scaled Q values (quant_q_scaled), held from the end of one item,
  // where the group's round for them is published, to the codes at the top of the next
  float qsc[QF ? D / 64 : 1][QF ? 32 : 1];
  int round = 0;
  auto fetch_q = [&](int id) {
    const int bh_ = id / nq, I_ = id - bh_ * nq;
    const int row = I_ * 128 + wq * 32 + (lane & 31);
    if constexpr (QF) {
      const int b_ = bh_ / H;
      AttnCtx<D, HAS_MASK, HAS_BIAS, true>::load_q16(qa, b_, bh_ - b_ * H, row, Sq, lane, rawnext);
    } else {
      const uint8_t* qp = q8 + ((int64_t)bh_ * nq * 128 + row) * D + 32 * (lane >> 5);
#pragma unroll
      for (int hh = 0; hh < D / 64; ++hh) {
        const v4i lo = *reinterpret_cast<const v4i*>(qp + 64 * hh);
        const v4i hi = *reinterpret_cast<const v4i*>(qp + 64 * hh + 16);
        qnext[hh] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
      sqnext = sq[(int64_t)bh_ * nq + I_];
    }
  };
  auto cx_scaled = [&](const uint4 (&raw)[QF ? D / 64 : 1][4], float (&f)[QF ? D / 64 : 1][QF ? 32 : 1]) {
    if constexpr (QF) return AttnCtx<D, HAS_MASK, HAS_BIAS, true>::template quant_q_scaled<ODT>(raw, qa.c, f);
    return 0.0f;
  };
  if (QF && threadIdx.x < 8) qgx[threadIdx.x >> 2].tag[threadIdx.x & 3] = -1;  // before the first barrier
  int loaded = -1;
  int p = ta;
  if (p < tb) {
    bool act;
    // in flight with the first head's K/V copies (the head change below waits for both)
    fetch_q(pair_item(p, act));
  }
  bool first = true;
  while (p < tb) {
    const int bh = p / nq;
    const int seg_end = min(tb, (bh + 1) * nq);
    if (bh != loaded) {
      // every wave is done with the previous head's tiles
      attn_barrier();
      const AttnCtx<D, HAS_MASK, HAS_BIAS, true> dc(nullptr, k8, v8t, nullptr, sk, key_mask, key_bias, H, Sk, nq,
                                                    bh * nq, wq, lane);
      for (int j = grp; j < nk; j += 2) {
        uint8_t* buf = smem + j * T::BUF;
        dc.dma_k(buf, j * 128);
        dc.dma_v(buf + T::KB, j * 128);
        dc.dma_aux(buf + T::KB + T::VB, j * 128, Sk);
      }
      if (threadIdx.x < D) svl[threadIdx.x] = sv[(int64_t)bh * D + threadIdx.x];
      wait_vm0();
      attn_barrier();
      loaded = bh;
    }
    if constexpr (QF) {
      // the first item's block maximum (later ones are published at the end of an item)
      if (first)
        attn_group_publish(cx_scaled(rawnext, qsc), &qgx[grp], wq, round, lane);
    }
    first = false;
    bool active;
    const int id = pair_item(p, active);
    AttnCtx<D, HAS_MASK, HAS_BIAS, true> cx(nullptr, k8, v8t, nullptr, sk, key_mask, key_bias, H, Sk, nq, id, wq,
                                            lane);
    if constexpr (QF) {
      // every wave, active or not, takes part in the group's round (published at the end of
      // the previous item); a stand-in item quantizes a real tile and writes no scale
      AttnQ16 qx = qa;
      if (!active) qx.sq_out = nullptr;
      cx.quant_q_codes(qsc, attn_group_gather(&qgx[grp], round), qx, nq);
      ++round;
    } else {
#pragma unroll
      for (int hh = 0; hh < D / 64; ++hh) cx.qf[hh] = qnext[hh];
      cx.sqI = sqnext;
    }
    const int np = p + 2 < seg_end ? p + 2 : seg_end;  // first tile of the next pair
    // the next pair's item, or this one again after the range's last pair (fetched, unused)
    bool nact;
    const int nid = np < tb ? pair_item(np, nact) : id;
    AttnState<D> st;
    if (active) {
      st.init();
      int j = (int)(((int64_t)cx.I * nk) / nq);
      // One KV tile; LAST: the item's last one, under whose products the next item's Q
      // loads (written out twice so that the fetched registers are live only there)
      auto kv_tile = [&](int i, auto last) {
        constexpr bool LAST = decltype(last)::value;
        // q8 / sq of the next item load under the last tile's products
        if constexpr (!QF && LAST) fetch_q(nid);
        const uint8_t* buf = smem + j * T::BUF;
        const float skj = cx.skh[j];
        const int kv0 = j * 128;
        v16f s[4];
        AttnPB<false> pb;
        AttnMfmaRun<D, 0, 0, 0, 4>::run(buf + T::KB, buf, fo, pb, cx.qf, s, st);
        if (attn_tile_needs_mask<HAS_MASK, HAS_BIAS>(buf + T::KB + T::VB, kv0, Sk, lane)) {
          // (not on the last tile, under which the next item's Q rows load: the fetched
          // registers live across the branch would not fit)
          if (!LAST && attn_tile_all_masked<HAS_MASK, HAS_BIAS>(buf + T::KB + T::VB, lane)) {
            j = j + 1 == nk ? 0 : j + 1;
            return;
          }
          attn_mask_scores<HAS_MASK, HAS_BIAS>(s, buf + T::KB + T::VB, kv0, Sk, cx.sqI, skj, lane);
        }
        // O and l are still zero on the first tile processed: rescaling them changes no bit
        attn_softmax_tile<HAS_BIAS>(s, cx.sqI, skj, 0u, i > 0, st, pb);
        // QF: the next item's 16-bit Q rows load under the last tile's PV products, once the
        // scores and the Q fragments are dead
        if constexpr (QF && LAST) fetch_q(nid);
        AttnMfmaRun<D, 0, 2, 0, 0>::run(buf + T::KB, buf, fo, pb, cx.qf, s, st);
        j = j + 1 == nk ? 0 : j + 1;
      };
      for (int i = 0; i < nk - 1; ++i) kv_tile(i, std::false_type{});
      kv_tile(nk - 1, std::true_type{});
    }
    // Every path fetches (an inactive group too), so the fetched registers are dead from
    // their use at the top of the loop to the fetch.
    if (!active) fetch_q(nid);
    const int row0 = cx.I * 128 + wq * 32;  // the wave's first query row
    if (active && row0 < Sq) {
      AttnSv<D> svr;
      svr.load_lds(svl, lane);
      if constexpr (STAGE) {
        // the next item's Q loads land while the rows are staged; after the wait nothing but
        // the stores is in flight at the top of the loop
        AttnStaged<D> rows;
        attn_stage_rows<D, ODT>(st, svr, lane, ostage + 2048 * wave, rows);
        wait_vm0();
        char* wrow0 =
            static_cast<char*>(out) + ((int64_t)cx.b * os_b + (int64_t)cx.h * os_h + (int64_t)row0 * os_s) * 2;
        attn_write_rows<D>(rows, wrow0, os_s * 2, os_d * 2, ovec, min(32, Sq - row0), lane);
      } else {
        wait_vm0();
        if (cx.qrow < Sq) attn_store<D, ODT>(st, svr, cx.b, cx.h, cx.qrow, lane, out, os_b, os_h, os_s, os_d);
      }
    } else {
      wait_vm0();
    }
    // QF: the next item's block maximum, published for the group's round at the top of the loop
    if constexpr (QF) attn_group_publish(cx_scaled(rawnext, qsc), &qgx[grp], wq, round, lane);
    p = np;
  }
}

// kv_mode MXF8_ATTN_KV_AUTO takes attn_fwd_resident_kernel whenever every KV tile of a head
// fits in LDS and no repair is asked for; MXF8_ATTN_KV_STREAM always takes attn_fwd_kernel.
template <int D, bool M_, bool B_, bool R_, int ODT>
static void launch_attn(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t, const float* sq, const float* sk,
                        const float* sv, const uint8_t* km, const float* kb, float tau, void* out,
                        const int64_t os[4], int64_t B, int64_t H, int64_t Sq, int64_t Sk, const AttnQ16* qa,
                        int kv_mode, hipStream_t st) {
  const int64_t nq = cdiv(Sq, 128);
  const int64_t nk = cdiv(Sk, 128);
  const int64_t total = nq * B * H;
  const AttnQ16 qv = qa != nullptr ? *qa : AttnQ16{nullptr, 0, 0, 0, 0.0f, nullptr};
  if (!R_ && kv_mode == MXF8_ATTN_KV_AUTO && nk <= AttnResident<D>::NKMAX) {
    const int cus = device_cus();
    const unsigned g = (unsigned)(cus > 0 && total > cus ? cus : total);
    if (qa != nullptr)
      attn_fwd_resident_kernel<D, M_, B_, ODT, true><<<dim3(g), 512, 0, st>>>(
          nullptr, k8, v8t, nullptr, sk, sv, km, kb, out, os[0], os[1], os[2], os[3], (int)H, (int)Sq, (int)Sk,
          (int)nq, (int)total, qv);
    else
      attn_fwd_resident_kernel<D, M_, B_, ODT, false><<<dim3(g), 512, 0, st>>>(
          q8, k8, v8t, sq, sk, sv, km, kb, out, os[0], os[1], os[2], os[3], (int)H, (int)Sq, (int)Sk, (int)nq,
          (int)total, qv);
    return;
  }
  const dim3 grid((unsigned)(nq * B * H));
  const uint32_t rep_add = R_ ? attn_repair_addend(tau) : 0u;
  if (qa != nullptr)
    attn_fwd_kernel<D, M_, B_, R_, ODT, true><<<grid, 256, 0, st>>>(
        nullptr, k8, v8t, nullptr, sk, sv, km, kb, rep_add, out, os[0], os[1], os[2], os[3], (int)H, (int)Sq, (int)Sk,
        (int)nq, qv);
  else
    attn_fwd_kernel<D, M_, B_, R_, ODT, false><<<grid, 256, 0, st>>>(
        q8, k8, v8t, sq, sk, sv, km, kb, rep_add, out, os[0], os[1], os[2], os[3], (int)H, (int)Sq, (int)Sk, (int)nq,
        qv);
}

// qa == nullptr: Q from q8 / sq; otherwise the fused Q quantizer reads qa.
template <int D, int ODT>
static void attn_dispatch_flags(bool hm, bool hb, bool rep, const uint8_t* q8, const uint8_t* k8,
                                const uint8_t* v8t, const float* sq, const float* sk, const float* sv,
                                const uint8_t* km, const float* kb, float tau, void* out, const int64_t os[4],
                                int64_t B, int64_t H, int64_t Sq, int64_t Sk, const AttnQ16* qa, int kv_mode,
                                hipStream_t st) {
#define MXF8_ATTN_CASE(M_, B_, R_)                                                                                \
  if (hm == M_ && hb == B_ && rep == R_) {                                                                        \
    launch_attn<D, M_, B_, R_, ODT>(q8, k8, v8t, sq, sk, sv, km, kb, tau, out, os, B, H, Sq, Sk, qa, kv_mode, st); \
    return;                                                                                                       \
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
                                 const AttnQ16* qa, int kv_mode, hipStream_t st)
MXF8_ATTN_DECL(128, 0);
MXF8_ATTN_DECL(128, 1);
MXF8_ATTN_DECL(64, 0);
MXF8_ATTN_DECL(64, 1);

}  // namespace mxf8
