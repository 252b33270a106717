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
// 8 waves on a 256 x 256 tile, two waves per SIMD, so that one wave's LDS reads and
// barrier waits overlap the other's matrix products.  Operand tiles are copied
// global -> LDS with the direct-to-LDS DMA (buffer_load_dwordx4 ... lds: 64 lanes x 16
// bytes into 1 KB of LDS) into two stage buffers; one barrier per stage publishes stage
// k and retires the buffer that stage k+1 is then loaded into, so the copy of stage k+1
// overlaps the MFMAs of stage k.  Inside a tile each 128-byte row holds 8 chunks of 16
// bytes stored at chunk ^ lds_swz(row), which makes the ds_read_b128 fragment reads
// bank-conflict free.
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

template <class C>
__device__ __forceinline__ void mma_stage(const uint8_t* stage, int wrow0, int xrow0, int lane,
                                          v16f (&acc)[C::TN][C::TM]) {
  const uint8_t* tW = stage;
  const uint8_t* tX = stage + C::BN * GEMM_BK;
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    const int c0 = 4 * kh + 2 * (lane >> 5);
    v8i af[C::TN], bf[C::TM];
#pragma unroll
    for (int t = 0; t < C::TN; ++t) af[t] = lds_frag(tW, wrow0 + 32 * t + (lane & 31), c0);
#pragma unroll
    for (int t = 0; t < C::TM; ++t) bf[t] = lds_frag(tX, xrow0 + 32 * t + (lane & 31), c0);
#pragma unroll
    for (int a = 0; a < C::TN; ++a)
#pragma unroll
      for (int b = 0; b < C::TM; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[a], bf[b], acc[a][b], 0, 0, 0, 0, 0, 0);
  }
}

template <class C, int ACT, bool HAS_LORA, bool KTAIL>
__global__ __launch_bounds__(C::THREADS) void gemm_fp8_rowwise_kernel(
    const uint8_t* __restrict__ a8, const uint8_t* __restrict__ w8, const float* __restrict__ sa,
    const float* __restrict__ sw, const uint16_t* __restrict__ bias, const uint16_t* __restrict__ lora_t,
    const uint16_t* __restrict__ lora_b, int lora_r, float lora_scale, uint16_t* __restrict__ out, int M, int N,
    int K, int64_t ld_out, int tiles_m, int tiles_n) {
  constexpr int TM = C::TM, TN = C::TN;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];

  int tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * C::BM, n0 = tn * C::BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wn = wave / C::WM, wm = wave % C::WM;

  // DMA: lane i of instruction J (stage rows 8J..8J+7) fills LDS bytes [16 i, 16 i + 16),
  // i.e. row 8J + i/8, physical chunk i%8, which must hold logical chunk
  // (i%8) ^ lds_swz(8J + i/8); that depends on the parity of J, hence two offsets.
  uint32_t lane_off[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    lane_off[par] = (uint32_t)((lane >> 3) * K + (((lane & 7) ^ lds_swz<GEMM_BK>(8 * par + (lane >> 3))) << 4));
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w8 + (int64_t)n0 * K), 0, (int)((int64_t)(N - n0) * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a8 + (int64_t)m0 * K), 0, (int)((int64_t)(M - m0) * K), 0x00020000);
  const int nk = (K + GEMM_BK - 1) / GEMM_BK;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  const int wrow0 = wn * (C::BN / C::WN), xrow0 = wm * (C::BM / C::WM);
  gemm_dma<C>(wrs, xrs, smem, lane_off, K, wave, 0);
  for (int ks = 0; ks < nk; ++ks) {
    uint8_t* cur = smem + (ks & 1) * C::STAGE;
    // Stage ks is this wave's only DMA in flight.  After the barrier every wave's copy of
    // stage ks has landed and every wave has finished stage ks-1, whose buffer then takes
    // stage ks+1 while stage ks is multiplied.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    block_barrier();
    if (KTAIL && ks == nk - 1) {
      zero_tail<C>(cur, (K % GEMM_BK) >> 4);
      block_barrier();
    }
    if (ks + 1 < nk) gemm_dma<C>(wrs, xrs, smem + ((ks + 1) & 1) * C::STAGE, lane_off, K, wave, (ks + 1) * GEMM_BK);
    mma_stage<C>(cur, wrow0, xrow0, lane, acc);
  }

  // ---- epilogue ------------------------------------------------------------------------
  // acc[a][b] register i: channel n = nb + 8 (i/4) + 4 g + i%4, token m = mb + lane%32.
  const int g = lane >> 5;
  const bool vec_ok = ((N & 3) == 0) && ((ld_out & 3) == 0) && ((((uintptr_t)bias) & 7) == 0) &&
                      ((((uintptr_t)out) & 7) == 0);
#pragma unroll
  for (int a = 0; a < TN; ++a) {
    const int nb = n0 + wrow0 + 32 * a;
    float swq[4][4], bq[4][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nb + 8 * q + 4 * g;
      if (vec_ok && n + 3 < N) {
        const v4f s4 = *reinterpret_cast<const v4f*>(sw + n);
        swq[q][0] = s4[0]; swq[q][1] = s4[1]; swq[q][2] = s4[2]; swq[q][3] = s4[3];
        if (bias) {
          const uint2 b4 = *reinterpret_cast<const uint2*>(bias + n);
          bq[q][0] = __uint_as_float(b4.x << 16); bq[q][1] = __uint_as_float(b4.x & 0xffff0000u);
          bq[q][2] = __uint_as_float(b4.y << 16); bq[q][3] = __uint_as_float(b4.y & 0xffff0000u);
        } else {
          bq[q][0] = bq[q][1] = bq[q][2] = bq[q][3] = 0.0f;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int nn = min(n + e, N - 1);
          swq[q][e] = sw[nn];
          bq[q][e] = bias ? bf16_bits_to_f32(bias[nn]) : 0.0f;
        }
      }
    }
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      const int m = m0 + xrow0 + 32 * b + (lane & 31);
      const float sam = sa[min(m, M - 1)];
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
            float v = acc[a][b][4 * q + e] * sam * swq[q][e] + bq[q][e];
            v = bf16r(v);
            if constexpr (HAS_LORA) {
              const float br = bf16r(bf16r(lacc[4 * q + e]) * lora_scale);
              v = bf16r(v + br);
            }
            if constexpr (ACT == MXF8_ACT_GELU_TANH) v = bf16r(gelu_tanh_f32(v));
            o[e] = f32_to_bf16_bits(v);
          }
          uint16_t* dst = out + (int64_t)m * ld_out + n;
          if (vec_ok && n + 3 < N) {
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

template <class C, int ACT, bool LORA, bool KTAIL>
static void launch_gemm(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                        const uint16_t* bias, const uint16_t* lt, const uint16_t* lb, int r, float ls, uint16_t* out,
                        int M, int N, int K, int64_t ld_out, hipStream_t st) {
  const int tiles_m = (int)cdiv(M, C::BM), tiles_n = (int)cdiv(N, C::BN);
  gemm_fp8_rowwise_kernel<C, ACT, LORA, KTAIL><<<dim3(tiles_m * tiles_n), dim3(C::THREADS), 0, st>>>(
      a8, w8, sa, sw, bias, lt, lb, r, ls, out, M, N, K, ld_out, tiles_m, tiles_n);
}

template <class C>
static void gemm_dispatch_tile(int act, bool lora, bool ktail, const uint8_t* a8, const uint8_t* w8,
                               const float* sa, const float* sw, const uint16_t* bias, const uint16_t* lt,
                               const uint16_t* lb, int r, float ls, uint16_t* out, int M, int N, int K,
                               int64_t ld_out, hipStream_t st) {
#define MXF8_GEMM_CASE(A, L, T)                                                                 \
  if (act == A && lora == L && ktail == T) {                                                    \
    launch_gemm<C, A, L, T>(a8, w8, sa, sw, bias, lt, lb, r, ls, out, M, N, K, ld_out, st); \
    return;                                                                                     \
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
    gemm_dispatch_tile<GemmBig>(act, lora, ktail, a8, w8, sa, sw, b16, lt, lb, (int)r, lora_scale, o16, iM, iN, iK,
                                 ld_out, stream);
  else
    gemm_dispatch_tile<GemmSmall>(act, lora, ktail, a8, w8, sa, sw, b16, lt, lb, (int)r, lora_scale, o16, iM, iN, iK,
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
