// Dense bf16 GEMM on MFMA for the shared expert and router projections of
// the prefill MoE block (fnx/engine.py:1786-1802 at more than four rows):
//
//   y[m, n] = bf16( sum_k a[m, k] * W[n, k] )   (F.linear, fp32 accumulation)
//
// a: bf16 rows of K (row m at a + m*lda), W: bf16 [N, K] row-major (the
// reference's Raw container), y: bf16 rows (row m at y + m*ldy).
//
// BM x BN output tiles per workgroup of 4 waves (2 x 2, each (BM/2) x (BN/2):
// TI x TJ v_mfma_f32_16x16x32_bf16 tiles). Both operands keep K contiguous,
// so a lane's MFMA fragment (8 consecutive k of one row of a, or of W) is one
// 16-byte piece: K runs in KC-wide chunks that stream straight into a ring of
// RING LDS slots by buffer-resource global->LDS DMA, RING - 1 chunks ahead,
// the 16-byte pieces of every row stored XOR-swizzled by row so the 16 rows a
// fragment read touches fall in different banks. One barrier per chunk.
// Workgroups that share rows of a run on one XCD. Products of two bf16 are
// exact in fp32, so the result is the rounding of an fp32 accumulation of
// exact terms.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BK = 32;  // k per MFMA step

// s_waitcnt with vmcnt <= N and lgkmcnt == 0 (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4] left at 7).
template <int N>
QMOE_DEV void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4));
}

template <int BM_, int BN_, int KC_, int RING_>
struct Bf16Tile {
  static constexpr int BM = BM_, BN = BN_, KC = KC_, RING = RING_;
  static constexpr int TI = BM / 32, TJ = BN / 32;
  static constexpr int NS = KC / BK;            // MFMA steps per chunk
  static constexpr int PPR = KC / 8;            // 16-byte pieces per row and chunk
  static constexpr int A_BYTES = BM * 2 * KC;
  static constexpr int B_BYTES = BN * 2 * KC;
  static constexpr int SLOT = A_BYTES + B_BYTES;
  static constexpr int AQ = A_BYTES / 1024 / 4;  // DMA instructions per wave and chunk (1 KB each)
  static constexpr int BQ = B_BYTES / 1024 / 4;
  static constexpr int IPC = AQ + BQ;
  static constexpr int LDS = RING * SLOT;
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "tile shape");
};

template <class T>
__global__ __launch_bounds__(kThreads) void bf16_gemm_kernel(const uint16_t* __restrict__ a, long lda,
                                                             const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                             long ldy, int M, int K, int N) {
  constexpr int BM = T::BM, BN = T::BN, KC = T::KC, RING = T::RING;
  constexpr int TI = T::TI, TJ = T::TJ, PPR = T::PPR;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int ntn = (N + BN - 1) / BN;
  const int ntiles = ((M + BM - 1) / BM) * ntn;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  if (tile >= ntiles) return;
  const int m0 = (tile / ntn) * BM, n0 = (tile % ntn) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave >> 1, wn = wave & 1;
  const int i16 = lane & 15, kb = lane >> 4;
  // piece swizzle of row r: the 16 rows of a fragment read spread over the banks
  auto swz = [](int r) { return PPR == 4 ? ((r >> 2) & 3) : (r & 7); };

  // ---- DMA sources: instruction q of wave w covers rows (64 / PPR) (4q + w)
  // + lane / PPR of its operand; LDS piece lane % PPR of the row holds k-piece
  // (lane % PPR) ^ swz(row). Rows past M or N re-read the last one (never
  // stored). Buffer resources bound every access to its tensor.
  constexpr int kRsrcWord3 = 0x00020000;
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc((void*)a, (short)0, (int)(((long)(M - 1) * lda + K) * 2), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, N * K * 2, kRsrcWord3);
  uint32_t aoff[T::AQ], boff[T::BQ];
#pragma unroll
  for (int q = 0; q < T::AQ; ++q) {
    const int r = (64 / PPR) * (4 * q + wave) + lane / PPR;
    aoff[q] = 2u * ((uint32_t)min(m0 + r, M - 1) * (uint32_t)lda + 8u * (uint32_t)((lane % PPR) ^ swz(r)));
  }
#pragma unroll
  for (int q = 0; q < T::BQ; ++q) {
    const int r = (64 / PPR) * (4 * q + wave) + lane / PPR;
    boff[q] = 2u * ((uint32_t)min(n0 + r, N - 1) * (uint32_t)K + 8u * (uint32_t)((lane % PPR) ^ swz(r)));
  }
  auto issue_chunk = [&](int c) {
    unsigned char* base = lds + (c % RING) * T::SLOT;
    const int k0 = c * KC;
#pragma unroll
    for (int q = 0; q < T::AQ; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (__attribute__((address_space(3))) void*)(base + (4 * q + wave_u) * 1024),
                                               16, (int)aoff[q], k0 * 2, 0, 0);
#pragma unroll
    for (int q = 0; q < T::BQ; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc_b, (__attribute__((address_space(3))) void*)(base + T::A_BYTES + (4 * q + wave_u) * 1024), 16,
          (int)boff[q], k0 * 2, 0, 0);
  };

  f32x4_v acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  int arow[TI], brow[TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i) arow[i] = wm * (BM / 2) + 16 * i + i16;
#pragma unroll
  for (int j = 0; j < TJ; ++j) brow[j] = wn * (BN / 2) + 16 * j + i16;

  const int nch = K / KC;
#pragma unroll
  for (int c = 0; c < RING - 1; ++c)
    if (c < nch) issue_chunk(c);
  for (int c = 0; c < nch; ++c) {
    // chunk c has landed once only the later chunks in flight may be pending
    if (c + RING - 2 < nch) wait_vm_lgkm0<(RING - 2) * T::IPC>();
    else __builtin_amdgcn_s_waitcnt(0);
    // every wave is past chunk c - 1: its ring slot takes chunk c + RING - 1.
    // A barrier without a fence: the wait above has settled what it orders,
    // and __syncthreads' fence would also wait for the chunks prefetched ahead.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + RING - 1 < nch) issue_chunk(c + RING - 1);
    const unsigned char* as = lds + (c % RING) * T::SLOT;
    const unsigned char* bs = as + T::A_BYTES;
#pragma unroll
    for (int st = 0; st < T::NS; ++st) {
      bf16x8_v bf[TJ];
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int r = brow[j];
        bf[j] = *reinterpret_cast<const bf16x8_v*>(bs + r * (2 * KC) + (((4 * st + kb) ^ swz(r)) << 4));
      }
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int r = arow[i];
        const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(as + r * (2 * KC) + (((4 * st + kb) ^ swz(r)) << 4));
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // lane holds column i16 of tile (i, j) for rows 4*kb + r
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + brow[j];
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * (BM / 2) + i * 16 + 4 * kb + r;
        if (m < M) y[(size_t)m * ldy + n] = (uint16_t)f32_to_bf16(acc[i][j][r]);
      }
    }
}

template <class T>
int launch_bf16_gemm(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N,
                     hipStream_t stream) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  if (dev < 0 || dev >= 64) return QMOE_EINVAL;
  static bool attr_set[64] = {};
  if (!attr_set[dev]) {
    err = hipFuncSetAttribute((const void*)bf16_gemm_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, T::LDS);
    if (err != hipSuccess) return (int)err;
    attr_set[dev] = true;
  }
  const long tiles = (long)((M + T::BM - 1) / T::BM) * ((N + T::BN - 1) / T::BN);
  const long blocks = (tiles + 7) / 8 * 8;  // whole XCD rounds (extra blocks exit)
  if (blocks > 0x7fffffffL) return QMOE_EINVAL;
  hipLaunchKernelGGL(bf16_gemm_kernel<T>, dim3((unsigned)blocks), dim3(kThreads), T::LDS, stream, (const uint16_t*)x,
                     ldx, (const uint16_t*)w, (uint16_t*)y, ldy, M, K, N);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int qmoe_bf16_gemm(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N, void* stream) {
  if (M < 1 || N < 1 || K < BK || (K % BK) || ldx < K || (ldx % 8) || ldy < N ||
      ((uintptr_t)x & 15) || ((uintptr_t)w & 15) ||
      ((long)(M - 1) * ldx + K) * 2 >= 0x80000000L || (long)N * K * 2 >= 0x80000000L)
    return QMOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  // 128 x 128 tiles where they give every CU two workgroups, else 128 x 64
  // (64-k chunks when K allows) where they give every CU one, else 64 x 64
  const long tiles128 = (long)((M + 127) / 128) * ((N + 63) / 64);
  const long tiles128x128 = (long)((M + 127) / 128) * ((N + 127) / 128);
  // 64-k chunks double-buffered where K allows (4096 x 3072 x 2048: 650 -> 980
  // TFLOP/s against 32-k chunks in a 4-slot ring: half the barriers and waits
  // per MFMA)
  if (tiles128x128 >= 512 && K % 64 == 0)
    return launch_bf16_gemm<Bf16Tile<128, 128, 64, 2>>(x, ldx, w, y, ldy, M, K, N, st);
  if (tiles128x128 >= 512) return launch_bf16_gemm<Bf16Tile<128, 128, 32, 4>>(x, ldx, w, y, ldy, M, K, N, st);
  if (tiles128 >= 256 && K % 64 == 0) return launch_bf16_gemm<Bf16Tile<128, 64, 64, 3>>(x, ldx, w, y, ldy, M, K, N, st);
  if (tiles128 >= 256) return launch_bf16_gemm<Bf16Tile<128, 64, 32, 4>>(x, ldx, w, y, ldy, M, K, N, st);
  return launch_bf16_gemm<Bf16Tile<64, 64, 32, 4>>(x, ldx, w, y, ldy, M, K, N, st);
}

}  // extern "C"
