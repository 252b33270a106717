// Row-wise scaled FP8 GEMM for gfx950 with a fused epilogue.
//
//   out[m, n] = bf16( sum_k a8[m,k] * w8[n,k] * sa[m] * sw[n] + bias[n] )  (+ LoRA) (+ GELU-tanh)
//
// Both operands are K-contiguous (activations [M,K], weights [N,K]), which is the layout
// the f8f6f4 MFMA wants for both sides.  The kernel computes the transposed tile
// C^T = W X^T so that a lane of the 32x32 accumulator layout owns one output row m and
// runs of 4 consecutive output columns n: the epilogue then writes 8-byte bf16 quads.
//
// Block tile BM (tokens) x BN (channels) x 128 (K stage) on WM x WN waves, each wave
// (BM/WM) x (BN/WN) built from v_mfma_f32_32x32x64_f8f6f4.  The large configuration runs
// 8 waves on a 256 x 256 tile, two waves per SIMD.  Operand tiles are copied global -> LDS
// with the direct-to-LDS DMA (buffer_load_dwordx4 ... lds: 64 lanes x 16 bytes = 8 rows x
// 128 bytes, whole cache lines) into two stage buffers.  One barrier per stage, in its
// middle: after stage k's last fragment read it publishes stage k+1 and retires stage k's
// buffer, which then takes stage k+2; the half-0 fragments of stage k+1 are read while
// stage k's second half of products runs.
// Each 128-byte row holds 8 chunks of 16 bytes stored at chunk ^ lds_swz(row), which
// makes the ds_read_b128 fragment reads bank-conflict free.
//
// The kernel is persistent: one workgroup per CU walks a sequence of output tiles.  The
// first stage of the next tile is copied while the current tile's epilogue runs, and the
// epilogue's channel scales, bias and token scales come from LDS (read into registers at
// the start of the tile), so neither the pipeline fill nor a workgroup launch separates
// two tiles.  A whole output tile (no LoRA) is staged through the freed stage buffer and
// written as 16-byte stores of whole row segments.
#include <type_traits>

#include "common.h"

namespace mxf8 {

constexpr int GEMM_BK = 128;

template <int BM_, int BN_, int WM_, int WN_>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NW = WM * WN;                        // waves per workgroup
  static constexpr int THREADS = 64 * NW;
  static constexpr int TM = BM / WM / 32;                   // 32x32 tiles per wave along m
  static constexpr int TN = BN / WN / 32;                   // along n
  static constexpr int STAGE = (BM + BN) * GEMM_BK;         // LDS bytes per stage (W tile, then X tile)
  static constexpr int DMA_PER_WAVE = (BM + BN) / 8 / NW;   // 1 KB DMA instructions per wave per stage
  static_assert((BN / 8) % DMA_PER_WAVE == 0, "a wave's DMA rows must lie in one operand");
  static_assert(DMA_PER_WAVE % 2 == 0, "DMA instruction parity must follow the loop index");
};
typedef GemmCfg<256, 256, 4, 2> GemmBig;    // 8 waves, 128 KB LDS, one workgroup per CU
typedef GemmCfg<128, 128, 2, 2> GemmSmall;  // 4 waves, 64 KB LDS, two workgroups per CU

__device__ __forceinline__ v8i lds_frag(const uint8_t* tile, int row, int chunk0) {
  // 32 bytes = logical chunks chunk0, chunk0 + 1 of `row` (swizzled storage)
  const int sw = lds_swz<GEMM_BK>(row);
  const v4i lo = *reinterpret_cast<const v4i*>(tile + row * GEMM_BK + ((chunk0 ^ sw) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(tile + row * GEMM_BK + (((chunk0 + 1) ^ sw) << 4));
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

__device__ __forceinline__ float gelu_tanh_f32(float z) {
  // 0.5 z (1 + tanh(u)) = z * sigmoid(2u),  u = sqrt(2/pi) (z + 0.044715 z^3)
  const float u2 = z * __builtin_fmaf(0.0713548162726f, z * z, 1.5957691216057308f);  // 2u
  const float e = __builtin_amdgcn_exp2f(-u2 * 1.4426950408889634f);
  return z * __builtin_amdgcn_rcpf(1.0f + e);
}


// fp32 -> bf16 -> fp32 and fp32 pair -> packed bf16 pair, both with the hardware
// round-to-nearest-even conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ float bf16r(float f) { return (float)(__bf16)f; }
__device__ __forceinline__ uint32_t bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
}
// bf16r of two values with one conversion: the low half moves up, the high half is masked
// (three instructions for two roundings instead of four)
__device__ __forceinline__ void bf16r2(float& a, float& b) {
  const uint32_t w = bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

// 16 bytes of an output tile.  Whole tiles leave with non-temporal stores: the kernel never
// reads them back, and streaming the lines out of the L2 early leaves it to the operand panels
// and makes the next kernels' reads wait less on write-backs.  Same process on MI355X: the
// 480p hot-path step 4.758 -> 4.696 ms, and a chained block (each output feeding the next
// kernel) 4.610 -> 4.556 ms; non-temporal attention-output stores, quantizer code stores or
// quantizer loads on top were each slower in the chained block.
__device__ __forceinline__ void store_out16(uint16_t* p, const uint4& v) {
  __builtin_nontemporal_store(v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w}, reinterpret_cast<v4i*>(p));
}

// Map a tile sequence number s to an output tile.  Workgroups are dealt to the 8 XCDs
// round-robin and a persistent workgroup b walks s = b, b + G, b + 2G, ... (G = grid, a
// multiple of 8), so s % 8 names the XCD: give every XCD a contiguous range of tile ids,
// then walk that range in groups of group_m token-tiles so concurrently running tiles
// share operand panels in the XCD's L2.
__device__ __forceinline__ void tile_coords(int s, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int nwg = tiles_m * tiles_n;
  const int q = nwg >> 3, rem = nwg & 7, x = s & 7, j = s >> 3;
  const int id = (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + j;
  const int per_group = group_m * tiles_n;
  const int g = id / per_group;
  const int first_m = g * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in = id - g * per_group;
  tm = first_m + in % gsize;
  tn = in / gsize;
}

// Workgroup barrier that waits for this wave's LDS traffic but, unlike __syncthreads(),
// not for its outstanding global->LDS DMA (which must stay in flight across it).
__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// This wave's share of one stage: DMA_PER_WAVE instructions of 8 rows x 128 bytes each,
// all from one operand (rows past the end of the operand read as zero: buffer range
// check).  Instruction J fills LDS stage rows [8J, 8J + 8): W rows for J < BN/8, X rows
// after.  `lane_off` holds the per-lane source offset for even and odd J.
template <class C>
__device__ __forceinline__ void gemm_dma(__amdgpu_buffer_rsrc_t wrs, __amdgpu_buffer_rsrc_t xrs, uint8_t* stage,
                                         const uint32_t (&lane_off)[2], int K, int wave, int k0) {
  const int J0 = wave * C::DMA_PER_WAVE;
  const bool is_w = J0 < C::BN / 8;
  const __amdgpu_buffer_rsrc_t rs = is_w ? wrs : xrs;
  const int row0 = is_w ? 8 * J0 : 8 * J0 - C::BN;  // first operand row of this wave's share
#pragma unroll
  for (int j = 0; j < C::DMA_PER_WAVE; ++j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_PTR(stage + (J0 + j) * 1024), 16, lane_off[j & 1],
                                             (row0 + 8 * j) * K + k0, 0, 0);
  }
}

// Zero the logical 16-byte chunks at or past K of every row of a stage (last, partial
// stage; K % 16 == 0).
template <class C>
__device__ __forceinline__ void zero_tail(uint8_t* stage, int valid_chunks) {
  for (int x = threadIdx.x; x < (C::BM + C::BN) * 8; x += C::THREADS) {
    const int row = x >> 3, c = x & 7;
    if (c >= valid_chunks)
      *reinterpret_cast<v4i*>(stage + row * GEMM_BK + ((c ^ lds_swz<GEMM_BK>(row)) << 4)) = v4i{0, 0, 0, 0};
  }
}

// One K stage of a wave's products in two halves (64 bytes of K each) around the stage's
// barrier.  Half 0 runs on A / B fragments read before it; after its products come the
// reads of half 1's fragments (each A fragment's registers take its half-1 fragment once
// its products have issued), so that every read of the stage is issued before the barrier.
template <class C>
__device__ __forceinline__ void mma_half0(const uint8_t* stage, int wrow0, int xrow0, int lane, v8i (&af)[C::TN],
                                          const v8i (&bf)[C::TM], v8i (&bf1)[C::TM], v16f (&acc)[C::TN][C::TM]) {
  const uint8_t* tW = stage;
  const uint8_t* tX = stage + C::BN * GEMM_BK;
  const int r = lane & 31, c1 = 4 + 2 * (lane >> 5);
#pragma unroll
  for (int t = 0; t < C::TM; ++t) bf1[t] = lds_frag(tX, xrow0 + 32 * t + r, c1);
#pragma unroll
  for (int a = 0; a < C::TN; ++a) {
#pragma unroll
    for (int b = 0; b < C::TM; ++b)
      acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[a], bf[b], acc[a][b], 0, 0, 0, 0, 0, 0);
    af[a] = lds_frag(tW, wrow0 + 32 * a + r, c1);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Half 1 of a stage (after its barrier).  The half-0 fragments of the following stage
// (`next`, landed) are read while these products run: B first (free since half 0), then
// each A fragment once its products have issued.
template <class C>
__device__ __forceinline__ void mma_half1(const uint8_t* next, int wrow0, int xrow0, int lane, v8i (&af)[C::TN],
                                          v8i (&bf)[C::TM], const v8i (&bf1)[C::TM], v16f (&acc)[C::TN][C::TM]) {
  const int r = lane & 31, c0 = 2 * (lane >> 5);
#pragma unroll
  for (int t = 0; t < C::TM; ++t) bf[t] = lds_frag(next + C::BN * GEMM_BK, xrow0 + 32 * t + r, c0);
#pragma unroll
  for (int a = 0; a < C::TN; ++a) {
#pragma unroll
    for (int b = 0; b < C::TM; ++b)
      acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[a], bf1[b], acc[a][b], 0, 0, 0, 0, 0, 0);
    af[a] = lds_frag(next, wrow0 + 32 * a + r, c0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ v8bf lds_chunk_bf16(const uint8_t* tile, int row, int chunk) {
  return *reinterpret_cast<const v8bf*>(tile + row * GEMM_BK + ((chunk ^ lds_swz<GEMM_BK>(row)) << 4));
}

// LoRA modes of the kernel: none, operands staged in LDS (r <= 128), or read from global
// memory in the epilogue (r > 128).
enum { LORA_NONE = 0, LORA_LDS = 1, LORA_GLOBAL = 2 };

// Column statistics of a fused QKV projection's K and V parts (the kernel's KVS mode): the
// attention's K quantizer needs the key mean over each batch item's whole sequence and the
// V quantizer the per-channel |max| over it (kernels/fp8_attention.py:338 and 140-155), so
// the epilogue emits both over the bf16 outputs it stores, per 128-row block of tokens:
//   part[0][p][c] = sum of out[m, kc0 + c],   part[1][p][c] = max |out[m, vc0 + c]|
// over the rows m of block p, [128 p, 128 p + 128), for every block that lies inside one batch
// item (S rows each) and below M.  The other blocks -- at most two per item, where an item
// boundary or M falls inside them -- are left to the consumer, which reads their rows.
// Fixed order throughout, so the statistics do not depend on scheduling.
struct KvStats {
  float* part;  // [2][nb][C] fp32
  int kc0;      // first key column, or -1 (no key sums)
  int vc0;      // first value column, or -1 (no value maxima)
  int C;        // columns of each part (heads x head dim), a multiple of 256
  int S;        // rows per batch item
  int nb;       // 128-row blocks, ceil(M / 128)
};
constexpr int KVS_BLOCK = 128;

// LoRA branch of one 32x32 output block from a LoRA chunk staged like a K stage (B rows
// [BN x 128 bytes], then t rows [BM x 128 bytes]; 64 rank columns in bf16):
// lacc^T[n][m] += sum_j B[n][j] t[m][j].  K step j reads logical chunk 2j + g of both.
template <class C>
__device__ __forceinline__ void lora_chunk_mma(const uint8_t* chunk, int wrow, int xrow, int g, v16f& lacc) {
#pragma unroll
  for (int j = 0; j < GEMM_BK / 32; ++j) {
    lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_chunk_bf16(chunk, wrow, 2 * j + g),
                                                   lds_chunk_bf16(chunk + C::BN * GEMM_BK, xrow, 2 * j + g), lacc,
                                                   0, 0, 0);
    // one K step's fragments at a time: the accumulators hold most of the registers
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Registers 4 q .. 4 q + 3 of an accumulator block.
__device__ __forceinline__ v4f quad4(const v16f& c, int q) {
  return v4f{c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]};
}

// LM (LoRA mode): with lora_t [M, r] = bf16(x A^T) and lora_b [N, r] = B, the epilogue adds
// the reference's LoRA branch bf16(bf16(t B^T) * lora_scale) to the bf16 linear output.
// In LORA_LDS mode the t and B tiles (r <= 128: one or two 64-column chunks) are copied
// like K stages: the first chunk during the last K stage, into the buffer the next tile's
// first stage would otherwise take; that stage then goes into the buffer the last K
// stage frees, so it still overlaps the epilogue.
// KVS (no LoRA, no activation): the K/V column statistics above, taken from the staged
// output rows of whole-channel tiles (the host guarantees N % 256 == 0, 16-byte rows).
template <class C, int ACT, int LM, bool KTAIL, bool KVS = false>
__global__ __launch_bounds__(C::THREADS) void gemm_fp8_rowwise_kernel(
    const uint8_t* __restrict__ a8, const uint8_t* __restrict__ w8, const float* __restrict__ sa,
    const float* __restrict__ sw, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ lora_t,
    const uint16_t* __restrict__ lora_b, int lora_r, float lora_scale, uint16_t* __restrict__ out, int M, int N,
    int K, int64_t ld_out, int tiles_m, int tiles_n, int group_m, KvStats kvs) {
  static_assert(!KVS || (LM == LORA_NONE && ACT == MXF8_ACT_NONE), "K/V statistics: plain epilogue only");
  static_assert(!KVS || C::WM * (C::BM / C::WM) == C::BM && C::BM / C::WM * 2 == KVS_BLOCK,
                "K/V statistics: two waves per 128-row block");
  constexpr int TM = C::TM, TN = C::TN;
  constexpr int EP_BYTES = (2 * C::BN + C::BM) * 4;  // channel scales, bias (fp32), token scales
  // with LoRA chunks in LDS: each wave's 2 KB output staging region (one 32 x 32 block)
  constexpr int LS_BYTES = LM == LORA_LDS ? C::NW * 2048 : 0;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE + EP_BYTES + LS_BYTES];
  static_assert(2 * C::STAGE + EP_BYTES + LS_BYTES <= 160 * 1024, "LDS exceeds the 160 KB of a CU");
  float* const ep_sw = reinterpret_cast<float*>(smem + 2 * C::STAGE);  // [BN]
  float* const ep_b = ep_sw + C::BN;                                   // [BN]
  float* const ep_sa = ep_b + C::BN;                                   // [BM]

  const int ntiles = tiles_m * tiles_n;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wn = wave / C::WM, wm = wave % C::WM;
  const int wrow0 = wn * (C::BN / C::WN), xrow0 = wm * (C::BM / C::WM);
  const int nk = (K + GEMM_BK - 1) / GEMM_BK;
  const int lrow = 2 * lora_r;  // LoRA operand row bytes
  // LoRA chunks (64 rank columns each) and the valid 16-byte chunks of the last one
  const int nl = LM == LORA_LDS ? (lora_r + 63) / 64 : 0;
  const int l_tail = LM == LORA_LDS ? ((lora_r & 63) * 2) >> 4 : 0;
  // DMA: lane i of instruction J (stage rows 8J..8J+7) fills LDS bytes [16 i, 16 i + 16),
  // i.e. row 8J + i/8, physical chunk i%8, which must hold logical chunk
  // (i%8) ^ lds_swz(8J + i/8); that depends on the parity of J, hence two offsets (per
  // source row stride: K bytes for the FP8 operands, 2r for the LoRA ones).
  uint32_t lane_off[2], lane_off_l[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const uint32_t c = (uint32_t)(((lane & 7) ^ lds_swz<GEMM_BK>(8 * par + (lane >> 3))) << 4);
    lane_off[par] = (uint32_t)((lane >> 3) * K) + c;
    lane_off_l[par] = LM == LORA_LDS ? (uint32_t)((lane >> 3) * lrow) + c : 0u;
  }
  // buffer resource over one tile's rows [row0, row0 + span) of an operand with `rows`
  // rows: rows past the end read as zero, and the byte range stays far below 2^31
  auto rsrc_s = [&](const void* base, int row0, int rows, int span, int stride) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)base + (int64_t)row0 * stride), 0,
                                             min(rows - row0, span) * stride, 0x00020000);
  };
  auto rsrc = [&](const uint8_t* base, int row0, int rows, int span) { return rsrc_s(base, row0, rows, span, K); };
  // LoRA chunk c of tile (tm, tn) -> stage buffer `dst` (rank bytes [128 c, 128 c + 128))
  auto lora_dma = [&](uint8_t* dst, int tm_, int tn_, int c) {
    gemm_dma<C>(rsrc_s(lora_b, tn_ * C::BN, N, C::BN, lrow), rsrc_s(lora_t, tm_ * C::BM, M, C::BM, lrow), dst,
                lane_off_l, lrow, wave, c * GEMM_BK);
  };
  static_assert(C::THREADS == C::BM + C::BN, "one thread per epilogue operand");

  int s = blockIdx.x;
  int tm, tn;
  tile_coords(s, tiles_m, tiles_n, group_m, tm, tn);
  __amdgpu_buffer_rsrc_t wrs = rsrc(w8, tn * C::BN, N, C::BN), xrs = rsrc(a8, tm * C::BM, M, C::BM);
  gemm_dma<C>(wrs, xrs, smem, lane_off, K, wave, 0);
  int gs = 0;  // global stage counter: stage buffer parity runs on across tiles

  for (; s < ntiles; s += gridDim.x) {
    const int m0 = tm * C::BM, n0 = tn * C::BN;
    // the tile's channel scales, bias and token scales, read now (their latency hides
    // behind the mainloop) and handed to the epilogue through LDS after it.  Thread t < BN
    // reads channel n0 + t, the next BM threads token m0 + t - BN; indices past the end read
    // the last element and are zeroed at the hand-over.  Nothing here waits for a load: a
    // wait issued now would also wait for the previous tile's output stores.
    // (Unconditional loads from valid addresses, selected when handed over: a load under a
    // condition makes the compiler wait for it at the end of the condition.)
    const bool ep_chan = (int)threadIdx.x < C::BN;
    const int ep_idx = ep_chan ? n0 + (int)threadIdx.x : m0 + (int)threadIdx.x - C::BN;
    const bool ep_ok = ep_idx < (ep_chan ? N : M);
    const float ep_v0 = *(ep_chan ? sw + min(ep_idx, N - 1) : sa + min(ep_idx, M - 1));
    const bool ep_hb = ep_chan && bias != nullptr;
    const uint16_t ep_bias = *(ep_hb ? bias + min(ep_idx, N - 1) : reinterpret_cast<const uint16_t*>(sw));
    // the next tile of this workgroup, whose first stage is copied during this epilogue
    const int s_next = s + gridDim.x;
    int tm_n = 0, tn_n = 0;
    if (s_next < ntiles) tile_coords(s_next, tiles_m, tiles_n, group_m, tm_n, tn_n);

    v16f acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

    // Barrier in the middle of each stage, after its last LDS read: the next stage has
    // landed everywhere (each wave waited for its share of the copy, issued one barrier
    // earlier) and this stage's buffer is free for the copy two stages ahead.  The next
    // stage's half-0 fragments are then read while this stage's half-1 products run, and
    // the barrier's wait overlaps the half-0 products in flight, so the matrix cores do not
    // stall on a fragment read after every barrier (a barrier at the top of each stage,
    // before its first reads, measured 2-5% slower; products and their order per
    // accumulator are the same).  The stage after the tile's last is the next tile's first
    // (or, with LoRA chunks in LDS, chunk 0), copied into the buffer the next tile's
    // mainloop starts on.  With a K tail, the last stage's missing chunks are zeroed after
    // it lands and before its first read.
    // Entering: stage 0 of this tile is the only copy in flight, into buffer gs & 1 (the
    // epilogue operands, older, aside).
    auto after_last = [&](uint8_t* dst) {
      if constexpr (LM == LORA_LDS) {
        lora_dma(dst, tm, tn, 0);
      } else {
        if (s_next < ntiles) {
          wrs = rsrc(w8, tn_n * C::BN, N, C::BN);
          xrs = rsrc(a8, tm_n * C::BM, M, C::BM);
          gemm_dma<C>(wrs, xrs, dst, lane_off, K, wave, 0);
        }
      }
    };
    wait_vm0();
    block_barrier();
    if (KTAIL && nk == 1) {
      zero_tail<C>(smem + (gs & 1) * C::STAGE, (K % GEMM_BK) >> 4);
      block_barrier();
    }
    if (nk > 1)
      gemm_dma<C>(wrs, xrs, smem + ((gs + 1) & 1) * C::STAGE, lane_off, K, wave, GEMM_BK);
    else
      after_last(smem + ((gs + 1) & 1) * C::STAGE);
    v8i af[TN], bf[TM], bf1[TM];
    {
      const uint8_t* cur = smem + (gs & 1) * C::STAGE;
      const int r = lane & 31, c0 = 2 * (lane >> 5);
#pragma unroll
      for (int a = 0; a < TN; ++a) af[a] = lds_frag(cur, wrow0 + 32 * a + r, c0);
#pragma unroll
      for (int b = 0; b < TM; ++b) bf[b] = lds_frag(cur + C::BN * GEMM_BK, xrow0 + 32 * b + r, c0);
    }
    // nk >= 1 (K >= 16): a do-while tells the compiler that the waits inside run before the
    // epilogue, which then waits for none of the loads issued before the mainloop (a wait
    // there would also wait for the next tile's first stage, in flight by then).
    int ks = 0;
    do {
      uint8_t* cur = smem + (gs & 1) * C::STAGE;
      uint8_t* nxt = smem + ((gs + 1) & 1) * C::STAGE;
      mma_half0<C>(cur, wrow0, xrow0, lane, af, bf, bf1, acc);
      if (ks + 1 < nk) {
        wait_vm0();
        block_barrier();
        if (KTAIL && ks + 2 == nk) {
          zero_tail<C>(nxt, (K % GEMM_BK) >> 4);
          block_barrier();
        }
        if (ks + 2 < nk)
          gemm_dma<C>(wrs, xrs, cur, lane_off, K, wave, (ks + 2) * GEMM_BK);
        else
          after_last(cur);
      }
      // (after the last stage the reads of `nxt` fetch nothing that is used: the next tile
      // reads its first fragments after its first barrier; one code path keeps the
      // accumulators in place)
      mma_half1<C>(nxt, wrow0, xrow0, lane, af, bf, bf1, acc);
      ++gs;
    } while (++ks < nk);

    // ---- LoRA chunks (LDS mode) ---------------------------------------------------------
    // chunk 0 is in buffer gs & 1; the last K stage's buffer (gs + 1) & 1 is free once
    // every wave has passed the barrier below
    uint8_t* const lch0 = smem + (gs & 1) * C::STAGE;
    uint8_t* const lch1 = smem + ((gs + 1) & 1) * C::STAGE;
    if constexpr (LM == LORA_LDS) {
      wait_vm0();
      block_barrier();
      if (nl == 2) {
        // second chunk (r > 64): its copy is exposed; the next tile's first stage waits
        // for the end of the epilogue
        lora_dma(lch1, tm, tn, 1);
        wait_vm0();
        block_barrier();
      } else if (s_next < ntiles) {
        wrs = rsrc(w8, tn_n * C::BN, N, C::BN);
        xrs = rsrc(a8, tm_n * C::BM, M, C::BM);
        gemm_dma<C>(wrs, xrs, lch1, lane_off, K, wave, 0);
      }
      if (l_tail) {
        // rank columns past r in the last chunk hold the next rows' values: zero them
        zero_tail<C>(nl == 2 ? lch1 : lch0, l_tail);
        block_barrier();
      }
    }

    // ---- epilogue ----------------------------------------------------------------------
    // (the previous tile's epilogue reads of these LDS words finished before the barrier
    // at the top of this tile's last stage)
    if (ep_chan) {
      ep_sw[threadIdx.x] = ep_ok ? ep_v0 : 0.0f;
      ep_b[threadIdx.x] = ep_ok && ep_hb ? bf16_bits_to_f32(ep_bias) : 0.0f;
    } else {
      ep_sa[threadIdx.x - C::BN] = ep_ok ? ep_v0 : 0.0f;
    }
    block_barrier();

    // acc[a][b] register i: channel n = nb + 8 (i/4) + 4 g + i%4, token m = mb + lane%32.
    const int g = lane >> 5;
    // The LoRA branch of block (a, b) (zero without LoRA).
    auto lora_block = [&](int a, int b) {
      v16f lacc;
      if constexpr (LM != LORA_NONE) {
#pragma unroll
        for (int i = 0; i < 16; ++i) lacc[i] = 0.0f;
      }
      const int nl_ = wrow0 + 32 * a, ml = xrow0 + 32 * b + (lane & 31);
      if constexpr (LM == LORA_LDS) {
        lora_chunk_mma<C>(lch0, nl_ + (lane & 31), ml, g, lacc);
        if (nl == 2) lora_chunk_mma<C>(lch1, nl_ + (lane & 31), ml, g, lacc);
      } else if constexpr (LM == LORA_GLOBAL) {
        // LoRA up-projection on the bf16 MFMA from global memory (r > 128)
        const uint16_t* brow = lora_b + (int64_t)min(n0 + nl_ + (lane & 31), N - 1) * lora_r + 8 * g;
        const uint16_t* trow = lora_t + (int64_t)min(m0 + ml, M - 1) * lora_r + 8 * g;
        for (int kk = 0; kk < lora_r; kk += 16) {
          const v8bf bo = *reinterpret_cast<const v8bf*>(brow + kk);
          const v8bf to = *reinterpret_cast<const v8bf*>(trow + kk);
          lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bo, to, lacc, 0, 0, 0);
        }
      }
      return lacc;
    };
    // Output values of accumulators x (registers 4 q .. 4 q + 3 of a block, whose LoRA
    // branch is lacc), packed as two bf16 pairs.
    auto out_quad = [&](const v4f x, int q, const v16f& lacc, float sam, const v4f& swq, const v4f& bq) {
      // the reference's roundings: bf16 linear output, bf16 branch, bf16 branch * scale,
      // bf16 sum; GELU-tanh acts on the bf16 result.  Values go through them in pairs
      // (bf16r2); the last rounding is the output packing itself.
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(x[e] * sam, swq[e], bq[e]);
#pragma unroll
      for (int h = 0; h < 4; h += 2) {
        if constexpr (LM != LORA_NONE || ACT == MXF8_ACT_GELU_TANH) bf16r2(v[h], v[h + 1]);
        if constexpr (LM != LORA_NONE) {
          float b0 = lacc[4 * q + h], b1 = lacc[4 * q + h + 1];
          bf16r2(b0, b1);
          // scale 1 (the runtime folds alpha / rank into B): bf16(b * 1) = b, so the product
          // and its rounding change no bit and are skipped
          if (lora_scale != 1.0f) {
            b0 *= lora_scale;
            b1 *= lora_scale;
            bf16r2(b0, b1);
          }
          v[h] += b0;
          v[h + 1] += b1;
          if constexpr (ACT == MXF8_ACT_GELU_TANH) bf16r2(v[h], v[h + 1]);
        }
        if constexpr (ACT == MXF8_ACT_GELU_TANH) {
          v[h] = gelu_tanh_f32(v[h]);
          v[h + 1] = gelu_tanh_f32(v[h + 1]);
        }
      }
      return make_uint2(bf16x2(v[0], v[1]), bf16x2(v[2], v[3]));
    };

    // (KVS: every tile is staged -- the host checks the row alignment and that N is a multiple
    // of 256 -- token-tail tiles included, whose rows past M are not stored)
    const bool staged = KVS || (((ld_out & 7) == 0) && ((((uintptr_t)out) & 15) == 0) && (m0 + C::BM <= M) &&
                                (n0 + C::BN <= N));
    if (staged && LM != LORA_LDS) {
      // Whole tile in range: each 32-token round of this wave goes through a private 8 KB
      // LDS region in the buffer of the last K stage (free after the barrier above; the
      // next tile's first copy into it waits for the barrier at the top of its first
      // stage), then leaves as 16-byte stores covering whole 32 TN-channel row segments.
      constexpr int RB = TN * 64;     // staged row bytes (32 TN bf16 channels)
      constexpr int NCH = RB / 16;    // 16-byte chunks per staged row (chunk c at c ^ row % NCH)
      constexpr int RPI = 64 / NCH;   // rows per 64-lane read
      static_assert(32 * RB <= C::STAGE / C::NW, "per-wave staging region");
      uint8_t* const wreg = smem + ((gs + 1) & 1) * C::STAGE + wave * (C::STAGE / C::NW);
      const int r = lane & 31;
      // KVS: kv = 1 on key columns (sums), 2 on value columns (|max|), 0 elsewhere (uniform
      // over the workgroup).  A lane reads channels n0 + wrow0 + 8 (lane % NCH) + [0, 8) of
      // its rows and keeps their running statistic (ks) when the wave's 128-row block lies
      // inside one batch item and below M (kvx = kv there, else 0: no statistic).
      int kv = 0, kvx = 0;
      float ks[8];
      if constexpr (KVS) {
        kv = kvs.kc0 >= 0 && n0 >= kvs.kc0 && n0 < kvs.kc0 + kvs.C   ? 1
             : kvs.vc0 >= 0 && n0 >= kvs.vc0 && n0 < kvs.vc0 + kvs.C ? 2
                                                                       : 0;
        const int b0 = (m0 + xrow0) & ~(KVS_BLOCK - 1);
        kvx = b0 + KVS_BLOCK <= min((b0 / kvs.S + 1) * kvs.S, M) ? kv : 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) ks[e] = 0.0f;
      }
      // One 32-token round: outputs -> LDS, then 16-byte rows out (rows past M are not stored
      // in KVS mode), folding each chunk into the statistic ST (0 none, 1 sum, 2 |max|).
      // The lane index behind the staging addresses is opaque to the compiler here, so the
      // ~24 per-lane addresses derived from it are recomputed in each tile's epilogue rather
      // than held in registers across the persistent loop (with the statistics live they would
      // not fit and would go to scratch, whose reloads wait for every store in flight).
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int rk = ln & 31, gk = ln >> 5;
      auto round = [&](int b, auto st_tag) {
        constexpr int ST = decltype(st_tag)::value;
        const float sam = ep_sa[xrow0 + 32 * b + rk];
#pragma unroll
        for (int a = 0; a < TN; ++a) {
          const v16f lacc = lora_block(a, b);
          const int nl_ = wrow0 + 32 * a;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint2*>(wreg + rk * RB + (((4 * a + q) ^ (rk & (NCH - 1))) << 4) + 8 * gk) =
                out_quad(quad4(acc[a][b], q), q, lacc, sam,
                         *reinterpret_cast<const v4f*>(ep_sw + nl_ + 8 * q + 4 * gk),
                         *reinterpret_cast<const v4f*>(ep_b + nl_ + 8 * q + 4 * gk));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < 32 / RPI; ++i) {
          const int row = i * RPI + ln / NCH, ch = ln % NCH;
          const uint4 val = *reinterpret_cast<const uint4*>(wreg + row * RB + ((ch ^ (row & (NCH - 1))) << 4));
          const int grow = m0 + xrow0 + 32 * b + row;
          if (!KVS || grow < M) store_out16(out + (int64_t)grow * ld_out + n0 + wrow0 + ch * 8, val);
          if constexpr (ST != 0) {
            const uint32_t w4[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float lo = __uint_as_float(w4[e] << 16), hi = __uint_as_float(w4[e] & 0xffff0000u);
              if constexpr (ST == 1) {
                ks[2 * e] += lo;
                ks[2 * e + 1] += hi;
              } else {
                ks[2 * e] = fmaxf(ks[2 * e], fabsf(lo));
                ks[2 * e + 1] = fmaxf(ks[2 * e + 1], fabsf(hi));
              }
            }
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      };
      if constexpr (!KVS) {
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const float sam = ep_sa[xrow0 + 32 * b + r];
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            const v16f lacc = lora_block(a, b);
            const int nl_ = wrow0 + 32 * a;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              *reinterpret_cast<uint2*>(wreg + r * RB + (((4 * a + q) ^ (r & (NCH - 1))) << 4) + 8 * g) =
                  out_quad(quad4(acc[a][b], q), q, lacc, sam,
                           *reinterpret_cast<const v4f*>(ep_sw + nl_ + 8 * q + 4 * g),
                           *reinterpret_cast<const v4f*>(ep_b + nl_ + 8 * q + 4 * g));
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
          for (int i = 0; i < 32 / RPI; ++i) {
            const int row = i * RPI + lane / NCH, ch = lane % NCH;
            const uint4 val = *reinterpret_cast<const uint4*>(wreg + row * RB + ((ch ^ (row & (NCH - 1))) << 4));
            store_out16(out + (int64_t)(m0 + xrow0 + 32 * b + row) * ld_out + n0 + wrow0 + ch * 8, val);
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
      } else {
        typedef std::integral_constant<int, 0> St0;
        typedef std::integral_constant<int, 1> St1;
        typedef std::integral_constant<int, 2> St2;
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          if (kvx == 0)
            round(b, St0{});
          else if (kvx == 1)
            round(b, St1{});
          else
            round(b, St2{});
        }
      }
      if constexpr (KVS) {
        if (kv != 0) {
          // Lanes with one lane % NCH read the same channels: combine them (a fixed
          // butterfly), then the two waves of each 128-row block through LDS (each wave's
          // own staging region, free now), in wave order.
          if (kvx != 0) {
#pragma unroll
            for (int off = NCH; off < 64; off <<= 1) {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float o = __shfl_xor(ks[e], off, 64);
                ks[e] = kvx == 1 ? ks[e] + o : fmaxf(ks[e], o);
              }
            }
            if (lane < NCH) {
              float* dst = reinterpret_cast<float*>(wreg) + 8 * lane;
              *reinterpret_cast<v4f*>(dst) = v4f{ks[0], ks[1], ks[2], ks[3]};
              *reinterpret_cast<v4f*>(dst + 4) = v4f{ks[4], ks[5], ks[6], ks[7]};
            }
          }
          block_barrier();
          // thread t: tile channel t of wave column t / (BN / WN); waves 2h, 2h + 1 of that
          // column hold 128-row block h of the tile
          constexpr int CPW = C::BN / C::WN;  // channels per wave
          const int t = threadIdx.x;
          if (t < C::BN) {
            const int wn_t = t / CPW, c_in = t % CPW;
            const int col0 = kv == 1 ? kvs.kc0 : kvs.vc0;
            float* const pst = kvs.part + (int64_t)(kv - 1) * kvs.nb * kvs.C + (n0 - col0 + t);
#pragma unroll
            for (int h = 0; h < C::BM / KVS_BLOCK; ++h) {
              const int p = (m0 >> 7) + h, b0 = p * KVS_BLOCK;
              if (b0 + KVS_BLOCK <= min((b0 / kvs.S + 1) * kvs.S, M)) {
                const float* ra = reinterpret_cast<const float*>(smem + ((gs + 1) & 1) * C::STAGE +
                                                                 (wn_t * C::WM + 2 * h) * (C::STAGE / C::NW)) + c_in;
                const float x0 = ra[0], x1 = ra[(C::STAGE / C::NW) / 4];
                pst[(int64_t)p * kvs.C] = kv == 1 ? x0 + x1 : fmaxf(x0, x1);
              }
            }
          }
        }
      }
    } else if (staged) {
      // LoRA chunks and the next tile's first stage fill both stage buffers: each 32 x 32
      // block goes through a private 2 KB region of its own and leaves as 16-byte stores
      // covering 64-byte row segments.
      uint8_t* const wreg = smem + 2 * C::STAGE + EP_BYTES + wave * 2048;
      const int r = lane & 31;
#pragma unroll
      for (int a = 0; a < TN; ++a) {
        const int nl_ = wrow0 + 32 * a;
        v4f swq[4], bq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          swq[q] = *reinterpret_cast<const v4f*>(ep_sw + nl_ + 8 * q + 4 * g);
          bq[q] = *reinterpret_cast<const v4f*>(ep_b + nl_ + 8 * q + 4 * g);
        }
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const v16f lacc = lora_block(a, b);
          const float sam = ep_sa[xrow0 + 32 * b + r];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint2*>(wreg + r * 64 + ((q ^ (r & 3)) << 4) + 8 * g) =
                out_quad(quad4(acc[a][b], q), q, lacc, sam, swq[q], bq[q]);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int row = 16 * i + lane / 4, ch = lane % 4;
            const uint4 val = *reinterpret_cast<const uint4*>(wreg + row * 64 + ((ch ^ (row & 3)) << 4));
            store_out16(out + (int64_t)(m0 + xrow0 + 32 * b + row) * ld_out + n0 + nl_ + ch * 8, val);
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
      }
    } else {
      const bool vec_ok = ((N & 3) == 0) && ((ld_out & 3) == 0) && ((((uintptr_t)out) & 7) == 0);
#pragma unroll
      for (int a = 0; a < TN; ++a) {
        const int nl_ = wrow0 + 32 * a;  // tile-local channel base
        v4f swq[4], bq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          swq[q] = *reinterpret_cast<const v4f*>(ep_sw + nl_ + 8 * q + 4 * g);
          bq[q] = *reinterpret_cast<const v4f*>(ep_b + nl_ + 8 * q + 4 * g);
        }
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const int ml = xrow0 + 32 * b + (lane & 31);
          const int m = m0 + ml;
          const v16f lacc = lora_block(a, b);
          if (m < M) {
            const float sam = ep_sa[ml];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int n = n0 + nl_ + 8 * q + 4 * g;
              const uint2 o = out_quad(quad4(acc[a][b], q), q, lacc, sam, swq[q], bq[q]);
              uint16_t* dst = out + (int64_t)m * ld_out + n;
              if (vec_ok && n + 3 < N) {
                *reinterpret_cast<uint2*>(dst) = o;
              } else {
                const uint16_t oo[4] = {(uint16_t)o.x, (uint16_t)(o.x >> 16), (uint16_t)o.y, (uint16_t)(o.y >> 16)};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  if (n + e < N) dst[e] = oo[e];
              }
            }
          }
        }
      }
    }
    if constexpr (LM == LORA_LDS) {
      if (nl == 2) {
        // both buffers held LoRA chunks: once every wave is done with them, copy the next
        // tile's first stage into buffer gs & 1, where its mainloop starts
        if (s_next < ntiles) {
          block_barrier();
          wrs = rsrc(w8, tn_n * C::BN, N, C::BN);
          xrs = rsrc(a8, tm_n * C::BM, M, C::BM);
          gemm_dma<C>(wrs, xrs, lch0, lane_off, K, wave, 0);
        }
      } else {
        ++gs;  // the next tile's first stage went into buffer (gs + 1) & 1
      }
    }
    tm = tm_n;
    tn = tn_n;
  }
}

// ---- LoRA down-projection t = bf16(x A^T): x [M,K] bf16, A [r,K] bf16 -> t [M,r] -----
// A workgroup computes BM = 32 W rows of t by up to 128 rank columns (blockIdx.y selects
// columns [128 y, 128 y + 128)) on W waves of 32 rows, RT accumulators of 32 columns each.
// K is consumed 64 elements (128 bytes per row) per stage: the x tile (BM rows) and the A
// tile (32 RT rows) are copied global -> LDS with the DMA in the GEMM's row layout, so the
// waves share one copy of A.  K step j of a stage reads logical chunk 2j + g of both
// operands (a consistent K permutation); a 32-row block's products and their order do not
// depend on W, so neither do the results.
// The pass is bound by how many bytes of x are in flight (the products are a few percent of
// the time): the stages form a ring as deep as one CU's 160 KB of LDS holds (one workgroup
// per CU), and the copy of stage ks + NS - 1 is issued while stage ks is consumed.  The
// host picks W so that the tiles come out in whole rounds over the CUs.
constexpr int LD_BM_MAX = 160;
template <int RT, int W>
struct LoraDown {
  static constexpr int BM = 32 * W, AR = 32 * RT, STAGE = (BM + AR) * GEMM_BK;
  // DMA instructions per wave and stage: 4 of x (8 rows each) and the A tile's 4 RT dealt
  // round-robin (waves below A_EXTRA take one more)
  static constexpr int A_LO = (4 * RT) / W, A_EXTRA = (4 * RT) % W;
  static constexpr int P_LO = 4 + A_LO, P_HI = P_LO + (A_EXTRA ? 1 : 0);
  static constexpr int NS_LDS = (160 * 1024) / STAGE, NS_CNT = 2 + 63 / P_HI;
  static constexpr int NS = NS_LDS < NS_CNT ? (NS_LDS < 8 ? NS_LDS : 8) : (NS_CNT < 8 ? NS_CNT : 8);
  static_assert(NS >= 3 && (NS - 2) * P_HI < 64, "ring depth");
};

template <int RT, int W>
__global__ __launch_bounds__(64 * W) void lora_down_kernel(const uint8_t* __restrict__ x, int ldxb,
                                                           const uint8_t* __restrict__ a, uint16_t* __restrict__ t,
                                                           int M, int K, int r) {
  using L = LoraDown<RT, W>;
  constexpr int BM = L::BM, AR = L::AR, STAGE = L::STAGE, NS = L::NS;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int m0 = blockIdx.x * BM, j0 = blockIdx.y * 128;
  const int Kb = 2 * K;
  const int nk = (K + 63) / 64;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(x + (int64_t)m0 * ldxb), 0, min(M - m0, BM) * ldxb, 0x00020000);
  const __amdgpu_buffer_rsrc_t ars =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a + (int64_t)j0 * Kb), 0, min(r - j0, AR) * Kb, 0x00020000);
  // lane i of a DMA instruction J fills tile row 8J + i/8, physical chunk i%8 = logical
  // chunk (i%8) ^ lds_swz(row); the swizzle depends on the parity of J
  uint32_t xoff[2], aoff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const uint32_t c = (uint32_t)(((lane & 7) ^ lds_swz<GEMM_BK>(8 * par + (lane >> 3))) << 4);
    xoff[par] = (uint32_t)((lane >> 3) * ldxb) + c;
    aoff[par] = (uint32_t)((lane >> 3) * Kb) + c;
  }
  auto dma = [&](uint8_t* st, int kb0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int J = 4 * wave + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, LDS_PTR(st + J * 1024), 16, xoff[J & 1], 8 * J * ldxb + kb0, 0,
                                               0);
    }
#pragma unroll
    for (int j = 0; j < L::A_LO + (L::A_EXTRA ? 1 : 0); ++j) {
      const int J = wave + W * j;
      if (j < L::A_LO || wave < L::A_EXTRA)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, LDS_PTR(st + BM * GEMM_BK + J * 1024), 16, aoff[J & 1],
                                                 8 * J * Kb + kb0, 0, 0);
    }
  };
  v16f acc[RT];
#pragma unroll
  for (int u = 0; u < RT; ++u)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[u][i] = 0.0f;
  const int g = lane >> 5, xr = 32 * wave + (lane & 31);
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) dma(smem + s * STAGE, s * GEMM_BK);
  int slot = 0;  // ks % NS
  for (int ks = 0; ks < nk; ++ks) {
    uint8_t* cur = smem + slot * STAGE;
    // this wave's copies in flight are stages ks .. min(ks + NS - 2, nk - 1), P_LO or P_HI
    // instructions each and nothing else; wait for stage ks (for all of them near the end).
    // After the barrier every wave's copy of stage ks has landed and every wave has finished
    // stage ks - 1, whose slot takes stage ks + NS - 1.
    if (ks + NS - 2 >= nk)
      wait_vm0();
    else if (L::A_EXTRA && wave < L::A_EXTRA)
      wait_vm<(NS - 2) * L::P_HI>();
    else
      wait_vm<(NS - 2) * L::P_LO>();
    block_barrier();
    if (ks == nk - 1 && (K & 63)) {
      // zero the chunks at or past K (they hold the next row's elements)
      const int valid = (K & 63) >> 3;
      for (int e = threadIdx.x; e < (BM + AR) * 8; e += 64 * W) {
        const int row = e >> 3, c = e & 7, trow = row < BM ? row : row - BM;
        if (c >= valid)
          *reinterpret_cast<v4i*>(cur + row * GEMM_BK + ((c ^ lds_swz<GEMM_BK>(trow)) << 4)) = v4i{0, 0, 0, 0};
      }
      block_barrier();
    }
    if (ks + NS - 1 < nk) dma(smem + (slot == 0 ? NS - 1 : slot - 1) * STAGE, (ks + NS - 1) * GEMM_BK);
    slot = slot + 1 == NS ? 0 : slot + 1;
    const uint8_t* tA = cur + BM * GEMM_BK;
#pragma unroll
    for (int j = 0; j < GEMM_BK / 32; ++j) {
      const v8bf xf = lds_chunk_bf16(cur, xr, 2 * j + g);
#pragma unroll
      for (int u = 0; u < RT; ++u)
        acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_chunk_bf16(tA, 32 * u + (lane & 31), 2 * j + g), xf,
                                                         acc[u], 0, 0, 0);
    }
  }
  // acc[u] is t^T: rank column j = j0 + 32 u + 8 (i/4) + 4 g + i%4, row m = m0 + xr
  const int m = m0 + xr;
  if (m >= M) return;
#pragma unroll
  for (int u = 0; u < RT; ++u)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = j0 + 32 * u + 8 * q + 4 * g;  // r % 16 == 0: j < r covers j + 3
      if (j < r) {
        const v16f& c = acc[u];
        *reinterpret_cast<uint2*>(t + (int64_t)m * r + j) =
            make_uint2(bf16x2(c[4 * q], c[4 * q + 1]), bf16x2(c[4 * q + 2], c[4 * q + 3]));
      }
    }
}


template <class C, int ACT, int LM, bool KTAIL, bool KVS = false>
static void launch_gemm(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                        const uint16_t* bias, const uint16_t* lt, const uint16_t* lb, int r, float ls, uint16_t* out,
                        int M, int N, int K, int64_t ld_out, hipStream_t st, const KvStats& kvs = KvStats{}) {
  const int tiles_m = (int)cdiv(M, C::BM), tiles_n = (int)cdiv(N, C::BN);
  const int ntiles = tiles_m * tiles_n;
  // Persistent grid: as many workgroups as stay resident (LDS decides: one per CU for the
  // 256 x 256 tile, two for 128 x 128), a multiple of the 8 XCDs.
  constexpr int per_cu = (160 * 1024) / (2 * C::STAGE + (2 * C::BN + C::BM) * 4);
  int grid = device_cus() * per_cu;
  grid = grid >= 8 ? grid & ~7 : ntiles;
  if (grid <= 0 || grid > ntiles) grid = ntiles;
  // Token-tiles per L2 group (measured on MI355X at M = 20280, one process): long-K products
  // (each panel 3 MB at K = 12288) share best in groups of 4 (MLP-down 584-586 us against 592
  // with 2 and 602 with 1), the K = 3072 ones in groups of 8 (out-projection and MLP-up 1-2%
  // ahead of 4 and 16; QKV within 1.5% from 4 to 16).
  const int group_m = K >= 8192 ? 4 : 8;
  gemm_fp8_rowwise_kernel<C, ACT, LM, KTAIL, KVS><<<dim3(grid), dim3(C::THREADS), 0, st>>>(
      a8, w8, sa, sw, bias, lt, lb, r, ls, out, M, N, K, ld_out, tiles_m, tiles_n, group_m, kvs);
}

template <class C>
static void gemm_dispatch_tile(int act, int lm, bool ktail, const uint8_t* a8, const uint8_t* w8,
                               const float* sa, const float* sw, const uint16_t* bias, const uint16_t* lt,
                               const uint16_t* lb, int r, float ls, uint16_t* out, int M, int N, int K,
                               int64_t ld_out, hipStream_t st) {
#define MXF8_GEMM_CASE(A, L, T)                                                                 \
  if (act == A && lm == L && ktail == T) {                                                      \
    launch_gemm<C, A, L, T>(a8, w8, sa, sw, bias, lt, lb, r, ls, out, M, N, K, ld_out, st); \
    return;                                                                                     \
  }
#define MXF8_GEMM_CASES(A, L) MXF8_GEMM_CASE(A, L, false) MXF8_GEMM_CASE(A, L, true)
  MXF8_GEMM_CASES(MXF8_ACT_NONE, LORA_NONE)
  MXF8_GEMM_CASES(MXF8_ACT_NONE, LORA_LDS)
  MXF8_GEMM_CASES(MXF8_ACT_NONE, LORA_GLOBAL)
  MXF8_GEMM_CASES(MXF8_ACT_GELU_TANH, LORA_NONE)
  MXF8_GEMM_CASES(MXF8_ACT_GELU_TANH, LORA_LDS)
  MXF8_GEMM_CASES(MXF8_ACT_GELU_TANH, LORA_GLOBAL)
#undef MXF8_GEMM_CASES
#undef MXF8_GEMM_CASE
}

}  // namespace mxf8

using namespace mxf8;

extern "C" int mxf8_gemm_rowwise(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                                 const void* bias, int act, const void* lora_t, const void* lora_b, int64_t r,
                                 float lora_scale, void* out, int64_t M, int64_t N, int64_t K, int64_t ld_out,
                                 hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0) return set_error(MXF8_EINVAL, "gemm_rowwise: negative shape");
  if (M == 0 || N == 0) return MXF8_OK;
  if (K == 0) return set_error(MXF8_EINVAL, "gemm_rowwise: K must be positive");
  if (!a8 || !w8 || !sa || !sw || !out) return set_error(MXF8_EINVAL, "gemm_rowwise: null pointer");
  if (K % 16) return set_error(MXF8_EINVAL, "gemm_rowwise: K=%lld must be a multiple of 16", (long long)K);
  if (ld_out < N) return set_error(MXF8_EINVAL, "gemm_rowwise: ld_out < N");
  if (act != MXF8_ACT_NONE && act != MXF8_ACT_GELU_TANH) return set_error(MXF8_EINVAL, "gemm_rowwise: bad act");
  // buffer ranges span one tile: 256 rows of K bytes (FP8) or 2r bytes (LoRA)
  if (M > 0x7fffffff / 2 || N > 0x7fffffff / 2 || K > (1 << 22))
    return set_error(MXF8_EINVAL, "gemm_rowwise: shape too large");
  const bool lora = lora_t != nullptr;
  if (lora) {
    if (!lora_b) return set_error(MXF8_EINVAL, "gemm_rowwise: lora_t without lora_b");
    if (r <= 0 || r % 16 || r > 4096)
      return set_error(MXF8_EINVAL, "gemm_rowwise: LoRA rank must be a positive multiple of 16 (<= 4096)");
    if (((uintptr_t)lora_t % 16) || ((uintptr_t)lora_b % 16))
      return set_error(MXF8_EINVAL, "gemm_rowwise: LoRA operands must be 16-byte aligned");
  }
  if (((uintptr_t)a8 % 16) || ((uintptr_t)w8 % 16))
    return set_error(MXF8_EINVAL, "gemm_rowwise: FP8 operands must be 16-byte aligned");
  const bool ktail = (K % GEMM_BK) != 0;
  const int lm = !lora ? LORA_NONE : (r <= 128 ? LORA_LDS : LORA_GLOBAL);
  const int iM = (int)M, iN = (int)N, iK = (int)K;
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  const uint16_t* lt = static_cast<const uint16_t*>(lora_t);
  const uint16_t* lb = static_cast<const uint16_t*>(lora_b);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  // 256x256 tiles when they fill the chip, 128x128 otherwise.
  const int64_t big_tiles = cdiv(M, 256) * cdiv(N, 256);
  if (big_tiles >= 2 * 256)
    gemm_dispatch_tile<GemmBig>(act, lm, ktail, a8, w8, sa, sw, b16, lt, lb, (int)r, lora_scale, o16, iM, iN, iK,
                                ld_out, stream);
  else
    gemm_dispatch_tile<GemmSmall>(act, lm, ktail, a8, w8, sa, sw, b16, lt, lb, (int)r, lora_scale, o16, iM, iN, iK,
                                  ld_out, stream);
  return check_launch("gemm_rowwise");
}

extern "C" int64_t mxf8_gemm_kv_stats_bytes(int64_t M, int64_t C) {
  if (M <= 0 || C <= 0) return 0;
  return 2 * cdiv(M, KVS_BLOCK) * C * (int64_t)sizeof(float);
}

extern "C" int mxf8_gemm_rowwise_kv_stats(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                                          const void* bias, void* out, int64_t M, int64_t N, int64_t K,
                                          int64_t ld_out, int64_t S, int64_t k_col0, int64_t v_col0, int64_t C,
                                          float* part, hipStream_t stream) {
  const char* what = "gemm_rowwise_kv_stats";
  if (M <= 0 || N <= 0 || K <= 0) return set_error(MXF8_EINVAL, "%s: empty or negative shape", what);
  if (!a8 || !w8 || !sa || !sw || !out || !part) return set_error(MXF8_EINVAL, "%s: null pointer", what);
  if (K % 16) return set_error(MXF8_EINVAL, "%s: K=%lld must be a multiple of 16", what, (long long)K);
  if (M > (1 << 30) || N > 0x7fffffff / 2 || K > (1 << 22)) return set_error(MXF8_EINVAL, "%s: shape too large", what);
  // whole 256-channel tiles and 16-byte output rows: every tile leaves through the staged stores
  if (N % 256 || ld_out < N || ld_out % 8 || ((uintptr_t)out % 16))
    return set_error(MXF8_EINVAL, "%s: N and ld_out must be multiples of 256 and 8 (ld_out >= N), out 16-byte "
                     "aligned", what);
  if (((uintptr_t)a8 % 16) || ((uintptr_t)w8 % 16) || ((uintptr_t)part % 16))
    return set_error(MXF8_EINVAL, "%s: a8, w8 and part must be 16-byte aligned", what);
  if (S < KVS_BLOCK || M % S)
    return set_error(MXF8_EINVAL, "%s: S=%lld must be >= %d and divide M=%lld", what, (long long)S, KVS_BLOCK,
                     (long long)M);
  if (C <= 0 || C % 256) return set_error(MXF8_EINVAL, "%s: C=%lld must be a positive multiple of 256", what,
                                          (long long)C);
  if (k_col0 < 0 && v_col0 < 0) return set_error(MXF8_EINVAL, "%s: neither key nor value columns given", what);
  for (const int64_t c0 : {k_col0, v_col0})
    if (c0 >= 0 && (c0 % 256 || c0 + C > N))
      return set_error(MXF8_EINVAL, "%s: a column range must start at a multiple of 256 and end by N", what);
  if (k_col0 >= 0 && v_col0 >= 0 && k_col0 < v_col0 + C && v_col0 < k_col0 + C)
    return set_error(MXF8_EINVAL, "%s: key and value column ranges overlap", what);
  KvStats kvs;
  kvs.part = part;
  kvs.kc0 = k_col0 < 0 ? -1 : (int)k_col0;
  kvs.vc0 = v_col0 < 0 ? -1 : (int)v_col0;
  kvs.C = (int)C;
  kvs.S = (int)S;
  kvs.nb = (int)cdiv(M, KVS_BLOCK);
  const int iM = (int)M, iN = (int)N, iK = (int)K;
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  const bool ktail = (K % GEMM_BK) != 0;
  // the tile choice of mxf8_gemm_rowwise, so the output is that entry point's bit for bit
  const bool big = cdiv(M, 256) * cdiv(N, 256) >= 2 * 256;
#define MXF8_KVS_LAUNCH(Cfg, T)                                                                                    \
  launch_gemm<Cfg, MXF8_ACT_NONE, LORA_NONE, T, true>(a8, w8, sa, sw, b16, nullptr, nullptr, 0, 0.0f, o16, iM, iN, \
                                                      iK, ld_out, stream, kvs)
  if (big) {
    if (ktail) MXF8_KVS_LAUNCH(GemmBig, true); else MXF8_KVS_LAUNCH(GemmBig, false);
  } else {
    if (ktail) MXF8_KVS_LAUNCH(GemmSmall, true); else MXF8_KVS_LAUNCH(GemmSmall, false);
  }
#undef MXF8_KVS_LAUNCH
  return check_launch(what);
}

extern "C" int mxf8_lora_down(const void* x, int64_t ldx, const void* a, void* t, int64_t M, int64_t K, int64_t r,
                              hipStream_t stream) {
  if (M < 0 || K <= 0 || r <= 0) return set_error(MXF8_EINVAL, "lora_down: bad shape");
  if (M == 0) return MXF8_OK;
  if (!x || !a || !t) return set_error(MXF8_EINVAL, "lora_down: null pointer");
  if (r % 16 || r > 4096) return set_error(MXF8_EINVAL, "lora_down: r must be a multiple of 16 and <= 4096");
  if (K % 8 || ldx % 8 || ldx < K || ((uintptr_t)x % 16) || ((uintptr_t)a % 16) || ((uintptr_t)t % 8))
    return set_error(MXF8_EINVAL, "lora_down: K, ldx must be multiples of 8 (ldx >= K) and operands aligned");
  // per-workgroup buffer ranges are up to 160 rows of x and 128 rows of A
  if (M > 0x7fffffff / 2 || ldx > 0x7fffffff / (2 * LD_BM_MAX) || K > 0x7fffffff / (2 * 128))
    return set_error(MXF8_EINVAL, "lora_down: shape too large");
  const int64_t col_blocks = cdiv(r, 128);
  // Rows per workgroup (32 W): with one workgroup per CU the busiest CU handles
  // ceil(tiles / CUs) tiles, so take the W with the fewest rows on it (ties: the larger
  // tile, fewer copies of A).  M = 77648 on 256 CUs: 160 rows, 486 tiles in 2 rounds,
  // against 607 tiles of 128 rows in 3.
  const int64_t cus = device_cus();
  if (cus <= 0) return set_error(MXF8_ELAUNCH, "lora_down: the device's compute-unit count is unavailable");
  int W = 5;
  int64_t best = INT64_MAX;
  for (int w = 5; w >= 2; --w) {
    const int64_t rows = cdiv(cdiv(M, 32 * w) * col_blocks, cus) * 32 * w;
    if (rows < best) best = rows, W = w;
  }
  const dim3 grid((unsigned)cdiv(M, 32 * W), (unsigned)col_blocks);
  const uint8_t* xb = static_cast<const uint8_t*>(x);
  const uint8_t* ab = static_cast<const uint8_t*>(a);
  uint16_t* t16 = static_cast<uint16_t*>(t);
  const int rs = (int)(r < 128 ? r : 128);  // rank columns per workgroup
  const int RT = (rs + 31) / 32;
  const int ldxb = (int)(2 * ldx);
#define MXF8_LORA_DOWN_CASE(rt, w)                                                                  \
  if (RT == rt && W == w) {                                                                         \
    lora_down_kernel<rt, w><<<grid, 64 * w, 0, stream>>>(xb, ldxb, ab, t16, (int)M, (int)K, (int)r); \
    return check_launch("lora_down");                                                               \
  }
#define MXF8_LORA_DOWN_CASES(rt) \
  MXF8_LORA_DOWN_CASE(rt, 2) MXF8_LORA_DOWN_CASE(rt, 3) MXF8_LORA_DOWN_CASE(rt, 4) MXF8_LORA_DOWN_CASE(rt, 5)
  MXF8_LORA_DOWN_CASES(1)
  MXF8_LORA_DOWN_CASES(2)
  MXF8_LORA_DOWN_CASES(3)
  MXF8_LORA_DOWN_CASES(4)
#undef MXF8_LORA_DOWN_CASES
#undef MXF8_LORA_DOWN_CASE
  return set_error(MXF8_EINVAL, "lora_down: no kernel for %d rank tiles, %d waves", RT, W);
}
