// Row-wise scaled FP8 GEMM for gfx950 with a fused epilogue.
//
//   out[m, n] = bf16( sum_k a8[m,k] * w8[n,k] * sa[m] * sw[n] + bias[n] )  (+ LoRA) (+ GELU-tanh)
//
// Both operands are K-contiguous (activations [M,K], weights [N,K]), which is the layout
// the f8f6f4 MFMA wants for both sides.  The kernel computes the transposed tile
// C^T = W X^T so that a lane of the 32x32 accumulator layout owns one output row m and
// runs of 4 consecutive output columns n: the epilogue then writes 8-byte bf16 quads.
//
// Block tile BM (tokens) x BN (channels) x 128 (K stage), 4 waves in a 2x2 grid, each wave
// (BM/2) x (BN/2) built from v_mfma_f32_32x32x64_f8f6f4.  Operand tiles are copied
// global -> LDS with the direct-to-LDS DMA (buffer_load_dwordx4 ... lds: 64 lanes x 16
// bytes into 1 KB of LDS), double-buffered in two separate LDS arrays so the loads of stage
// k+1 overlap the MFMAs of stage k.  Inside a tile each 128-byte row holds 8 chunks of
// 16 bytes stored at chunk ^ (row & 7), which makes both the DMA writes and the
// ds_read_b128 fragment reads bank-conflict free.
#include "common.h"

namespace mxf8 {

constexpr int GEMM_BK = 128;

__device__ __forceinline__ v8i lds_frag(const uint8_t* tile, int row, int chunk0) {
  // 32 bytes = logical chunks chunk0, chunk0 + 1 of `row` (swizzled storage)
  const int sw = row & 7;
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

__device__ __forceinline__ float bf16r(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }

// Map the launch index to an output tile: first give every XCD a contiguous range of
// tile ids (workgroups are dealt to the 8 XCDs round-robin), then walk that range in
// groups of GROUP_M token-tiles so concurrently running tiles share operand panels in L2.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nwg = tiles_m * tiles_n;
  const int i = blockIdx.x;
  const int q = nwg >> 3, rem = nwg & 7, x = i & 7, j = i >> 3;
  const int id = (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + j;
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * tiles_n;
  const int g = id / per_group;
  const int first_m = g * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
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

// Copy ROWS x 128 bytes (rows [row0, row0+ROWS) of a K-contiguous operand, K offset k0)
// into a swizzled LDS tile; this wave's share is rows [wave*ROWS/4, (wave+1)*ROWS/4).
// Rows past the end of the operand read as zero (buffer range check).
template <int ROWS>
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, uint32_t lane_off, int K,
                                         int wave, int k0) {
#pragma unroll
  for (int j = 0; j < ROWS / 32; ++j) {
    const int r = wave * (ROWS / 4) + 8 * j;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, LDS_PTR(lds + r * GEMM_BK), 16,
                                             lane_off + (uint32_t)(r * K + k0), 0, 0, 0);
  }
}

// Zero the logical 16-byte chunks at or past K (last, partial stage; K % 16 == 0).
template <int ROWS>
__device__ __forceinline__ void zero_tail(uint8_t* lds, int valid_chunks) {
  for (int x = threadIdx.x; x < ROWS * 8; x += 256) {
    const int row = x >> 3, c = x & 7;
    if (c >= valid_chunks) *reinterpret_cast<v4i*>(lds + row * GEMM_BK + ((c ^ (row & 7)) << 4)) = v4i{0, 0, 0, 0};
  }
}

template <int TN, int TM>
__device__ __forceinline__ void mma_stage(const uint8_t* tW, const uint8_t* tX, int wrow0, int xrow0, int lane,
                                          v16f (&acc)[TN][TM]) {
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    const int c0 = 4 * kh + 2 * (lane >> 5);
    v8i af[TN], bf[TM];
#pragma unroll
    for (int t = 0; t < TN; ++t) af[t] = lds_frag(tW, wrow0 + 32 * t + (lane & 31), c0);
#pragma unroll
    for (int t = 0; t < TM; ++t) bf[t] = lds_frag(tX, xrow0 + 32 * t + (lane & 31), c0);
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[a], bf[b], acc[a][b], 0, 0, 0, 0, 0, 0);
  }
}

template <int BM, int BN, int ACT, bool HAS_LORA, bool KTAIL>
__global__ __launch_bounds__(256, 1) void gemm_fp8_rowwise_kernel(
    const uint8_t* __restrict__ a8, const uint8_t* __restrict__ w8, const float* __restrict__ sa,
    const float* __restrict__ sw, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ lora_t,
    const uint16_t* __restrict__ lora_b, int lora_r, float lora_scale, uint16_t* __restrict__ out, int M, int N,
    int K, int64_t ld_out, int tiles_m, int tiles_n) {
  constexpr int TM = BM / 64;  // 32x32 tiles per wave along m
  constexpr int TN = BN / 64;  // along n
  __shared__ __attribute__((aligned(1024))) uint8_t sW0[BN * GEMM_BK];
  __shared__ __attribute__((aligned(1024))) uint8_t sX0[BM * GEMM_BK];
  __shared__ __attribute__((aligned(1024))) uint8_t sW1[BN * GEMM_BK];
  __shared__ __attribute__((aligned(1024))) uint8_t sX1[BM * GEMM_BK];

  int tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wn = wave >> 1, wm = wave & 1;

  // DMA: lane i of an 8-row instruction fills LDS bytes [16 i, 16 i + 16), i.e. row i/8,
  // physical chunk i%8, which must hold logical chunk (i%8) ^ (i/8).
  const uint32_t lane_off = (uint32_t)((lane >> 3) * K + (((lane & 7) ^ (lane >> 3)) << 4));
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w8 + (int64_t)n0 * K), 0, (int)((int64_t)(N - n0) * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a8 + (int64_t)m0 * K), 0, (int)((int64_t)(M - m0) * K), 0x00020000);
  const int nk = (K + GEMM_BK - 1) / GEMM_BK;
  const int tail_chunks = (K % GEMM_BK) >> 4;
  constexpr int PER_STAGE = BN / 32 + BM / 32;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  const int wrow0 = wn * (BN / 2), xrow0 = wm * (BM / 2);
  // Steady state: two stages per iteration, buffer 0 then buffer 1, while at least three
  // stages remain; the last one or two stages (and the K tail) are peeled below so the
  // loop body has no data-dependent control flow.
  dma_tile<BN>(wrs, sW0, lane_off, K, wave, 0);
  dma_tile<BM>(xrs, sX0, lane_off, K, wave, 0);
  int ks = 0;
  for (; ks + 2 < nk; ks += 2) {
    dma_tile<BN>(wrs, sW1, lane_off, K, wave, (ks + 1) * GEMM_BK);
    dma_tile<BM>(xrs, sX1, lane_off, K, wave, (ks + 1) * GEMM_BK);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_STAGE) : "memory");
    block_barrier();
    mma_stage<TN, TM>(sW0, sX0, wrow0, xrow0, lane, acc);
    block_barrier();
    dma_tile<BN>(wrs, sW0, lane_off, K, wave, (ks + 2) * GEMM_BK);
    dma_tile<BM>(xrs, sX0, lane_off, K, wave, (ks + 2) * GEMM_BK);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_STAGE) : "memory");
    block_barrier();
    mma_stage<TN, TM>(sW1, sX1, wrow0, xrow0, lane, acc);
    block_barrier();
  }
  // stage ks is in flight into buffer 0
  const bool two_left = ks + 1 < nk;
  if (two_left) {
    dma_tile<BN>(wrs, sW1, lane_off, K, wave, (ks + 1) * GEMM_BK);
    dma_tile<BM>(xrs, sX1, lane_off, K, wave, (ks + 1) * GEMM_BK);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_STAGE) : "memory");
    block_barrier();
    mma_stage<TN, TM>(sW0, sX0, wrow0, xrow0, lane, acc);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  block_barrier();
  uint8_t* lW = two_left ? sW1 : sW0;
  uint8_t* lX = two_left ? sX1 : sX0;
  if (KTAIL) {
    zero_tail<BN>(lW, tail_chunks);
    zero_tail<BM>(lX, tail_chunks);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    block_barrier();
  }
  mma_stage<TN, TM>(lW, lX, wrow0, xrow0, lane, acc);

  // ---- epilogue ------------------------------------------------------------------------
  const int g = lane >> 5;
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = m0 + wm * (BM / 2) + 32 * b + (lane & 31);
    const float sam = sa[min(m, M - 1)];
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      const int nb = n0 + wn * (BN / 2) + 32 * a;
      v16f lacc;
      if constexpr (HAS_LORA) {
        // LoRA up-projection on the bf16 MFMA: lacc^T[n][m] = sum_j B[n][j] t[m][j]
#pragma unroll
        for (int i = 0; i < 16; ++i) lacc[i] = 0.0f;
        const uint16_t* brow = lora_b + (int64_t)min(nb + (lane & 31), N - 1) * lora_r + 8 * g;
        const uint16_t* trow = lora_t + (int64_t)min(m, M - 1) * lora_r + 8 * g;
        for (int kk = 0; kk < lora_r; kk += 16) {
          const v8bf bo = *reinterpret_cast<const v8bf*>(brow + kk);
          const v8bf to = *reinterpret_cast<const v8bf*>(trow + kk);
          lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bo, to, lacc, 0, 0, 0);
        }
      }
      if (m < M) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = nb + 8 * q + 4 * g;
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int nn = min(n + e, N - 1);
            float v = acc[a][b][4 * q + e] * sam * sw[nn];
            if (bias) v += bf16_bits_to_f32(bias[nn]);
            v = bf16r(v);
            if constexpr (HAS_LORA) {
              const float br = bf16r(bf16r(lacc[4 * q + e]) * lora_scale);
              v = bf16r(v + br);
            }
            if constexpr (ACT == MXF8_ACT_GELU_TANH) v = bf16r(gelu_tanh_f32(v));
            o[e] = f32_to_bf16_bits(v);
          }
          uint16_t* dst = out + (int64_t)m * ld_out + n;
          if (n + 3 < N && ((ld_out & 3) == 0)) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N) dst[e] = (uint16_t)o[e];
          }
        }
      }
    }
  }
}

// ---- LoRA down-projection t = bf16(x A^T): x [M,K] bf16, A [r,K] bf16 -> t [M,r] -----
// One wave per 32 rows of x and all r columns (r/32 accumulators, r <= 128).  K is
// consumed 64 at a time; lane group g holds the contiguous elements [32 g, 32 g + 32) of
// that slice for both operands (a consistent K permutation, so the sum is unchanged).
template <int RT>
__global__ __launch_bounds__(256) void lora_down_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                        const uint16_t* __restrict__ a, uint16_t* __restrict__ t,
                                                        int M, int K, int r) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m0 = (blockIdx.x * 4 + wave) * 32;
  if (m0 >= M) return;
  const int g = lane >> 5;
  const uint16_t* xr = x + (int64_t)min(m0 + (lane & 31), M - 1) * ldx + 32 * g;
  const uint16_t* ar[RT];
#pragma unroll
  for (int u = 0; u < RT; ++u) ar[u] = a + (int64_t)min(32 * u + (lane & 31), r - 1) * K + 32 * g;
  v16f acc[RT];
#pragma unroll
  for (int u = 0; u < RT; ++u)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[u][i] = 0.0f;
  const bool k64 = (K % 64) == 0;
  for (int k0 = 0; k0 < K; k0 += 64) {
    v8bf xo[4], ao[RT][4];
    const bool full = k64 || (k0 + 64 <= K);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kk = k0 + 32 * g + 8 * c;  // this lane's 8 elements
      if (full || kk + 8 <= K) {
        xo[c] = *reinterpret_cast<const v8bf*>(xr + k0 + 8 * c);
#pragma unroll
        for (int u = 0; u < RT; ++u) ao[u][c] = *reinterpret_cast<const v8bf*>(ar[u] + k0 + 8 * c);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xo[c][e] = (__bf16)0.0f;
#pragma unroll
          for (int u = 0; u < RT; ++u) ao[u][c][e] = (__bf16)0.0f;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int u = 0; u < RT; ++u) acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao[u][c], xo[c], acc[u], 0, 0, 0);
  }
  // acc[u] is t^T: rows j = 32u + 8(i/4) + 4g + i%4, column m = m0 + lane%32
  const int m = m0 + (lane & 31);
  if (m >= M) return;
#pragma unroll
  for (int u = 0; u < RT; ++u)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = 32 * u + 8 * (i >> 2) + 4 * g + (i & 3);
      if (j < r) t[(int64_t)m * r + j] = (uint16_t)f32_to_bf16_bits(acc[u][i]);
    }
}

template <int BM, int BN, int ACT, bool LORA, bool KTAIL>
static void launch_gemm(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                        const uint16_t* bias, const uint16_t* lt, const uint16_t* lb, int r, float ls, uint16_t* out,
                        int M, int N, int K, int64_t ld_out, hipStream_t st) {
  const int tiles_m = (int)cdiv(M, BM), tiles_n = (int)cdiv(N, BN);
  gemm_fp8_rowwise_kernel<BM, BN, ACT, LORA, KTAIL><<<dim3(tiles_m * tiles_n), dim3(256), 0, st>>>(
      a8, w8, sa, sw, bias, lt, lb, r, ls, out, M, N, K, ld_out, tiles_m, tiles_n);
}

template <int BM, int BN>
static void gemm_dispatch_tile(int act, bool lora, bool ktail, const uint8_t* a8, const uint8_t* w8,
                               const float* sa, const float* sw, const uint16_t* bias, const uint16_t* lt,
                               const uint16_t* lb, int r, float ls, uint16_t* out, int M, int N, int K,
                               int64_t ld_out, hipStream_t st) {
#define MXF8_GEMM_CASE(A, L, T)                                                                  \
  if (act == A && lora == L && ktail == T) {                                                     \
    launch_gemm<BM, BN, A, L, T>(a8, w8, sa, sw, bias, lt, lb, r, ls, out, M, N, K, ld_out, st); \
    return;                                                                                      \
  }
  MXF8_GEMM_CASE(MXF8_ACT_NONE, false, false)
  MXF8_GEMM_CASE(MXF8_ACT_NONE, false, true)
  MXF8_GEMM_CASE(MXF8_ACT_NONE, true, false)
  MXF8_GEMM_CASE(MXF8_ACT_NONE, true, true)
  MXF8_GEMM_CASE(MXF8_ACT_GELU_TANH, false, false)
  MXF8_GEMM_CASE(MXF8_ACT_GELU_TANH, false, true)
  MXF8_GEMM_CASE(MXF8_ACT_GELU_TANH, true, false)
  MXF8_GEMM_CASE(MXF8_ACT_GELU_TANH, true, true)
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
  if (M > 0x7fffffff / 2 || N > 0x7fffffff / 2 || K > 0x7fffffff / 2)
    return set_error(MXF8_EINVAL, "gemm_rowwise: shape too large");
  const bool lora = lora_t != nullptr;
  if (lora) {
    if (!lora_b) return set_error(MXF8_EINVAL, "gemm_rowwise: lora_t without lora_b");
    if (r <= 0 || r % 16 || r > 4096) return set_error(MXF8_EINVAL, "gemm_rowwise: LoRA rank must be a positive multiple of 16");
    if (((uintptr_t)lora_t % 16) || ((uintptr_t)lora_b % 16))
      return set_error(MXF8_EINVAL, "gemm_rowwise: LoRA operands must be 16-byte aligned");
  }
  if (((uintptr_t)a8 % 16) || ((uintptr_t)w8 % 16))
    return set_error(MXF8_EINVAL, "gemm_rowwise: FP8 operands must be 16-byte aligned");
  const bool ktail = (K % GEMM_BK) != 0;
  const int iM = (int)M, iN = (int)N, iK = (int)K;
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  const uint16_t* lt = static_cast<const uint16_t*>(lora_t);
  const uint16_t* lb = static_cast<const uint16_t*>(lora_b);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  // 256x256 tiles when they fill the chip, 128x128 otherwise.
  const int64_t big_tiles = cdiv(M, 256) * cdiv(N, 256);
  if (big_tiles >= 2 * 256)
    gemm_dispatch_tile<256, 256>(act, lora, ktail, a8, w8, sa, sw, b16, lt, lb, (int)r, lora_scale, o16, iM, iN, iK,
                                 ld_out, stream);
  else
    gemm_dispatch_tile<128, 128>(act, lora, ktail, a8, w8, sa, sw, b16, lt, lb, (int)r, lora_scale, o16, iM, iN, iK,
                                 ld_out, stream);
  return check_launch("gemm_rowwise");
}

extern "C" int mxf8_lora_down(const void* x, int64_t ldx, const void* a, void* t, int64_t M, int64_t K, int64_t r,
                              hipStream_t stream) {
  if (M < 0 || K <= 0 || r <= 0) return set_error(MXF8_EINVAL, "lora_down: bad shape");
  if (M == 0) return MXF8_OK;
  if (!x || !a || !t) return set_error(MXF8_EINVAL, "lora_down: null pointer");
  if (r % 16 || r > 128) return set_error(MXF8_EINVAL, "lora_down: r must be a multiple of 16 and <= 128");
  if (K % 8 || ldx % 8 || ((uintptr_t)x % 16) || ((uintptr_t)a % 16))
    return set_error(MXF8_EINVAL, "lora_down: K, ldx must be multiples of 8 and operands 16-byte aligned");
  if (M > 0x7fffffff / 2 || K > 0x7fffffff / 2) return set_error(MXF8_EINVAL, "lora_down: shape too large");
  const dim3 grid((unsigned)cdiv(M, 128));
  const uint16_t* x16 = static_cast<const uint16_t*>(x);
  const uint16_t* a16 = static_cast<const uint16_t*>(a);
  uint16_t* t16 = static_cast<uint16_t*>(t);
  if (r <= 32)
    lora_down_kernel<1><<<grid, 256, 0, stream>>>(x16, ldx, a16, t16, (int)M, (int)K, (int)r);
  else if (r <= 64)
    lora_down_kernel<2><<<grid, 256, 0, stream>>>(x16, ldx, a16, t16, (int)M, (int)K, (int)r);
  else
    lora_down_kernel<4><<<grid, 256, 0, stream>>>(x16, ldx, a16, t16, (int)M, (int)K, (int)r);
  return check_launch("lora_down");
}
