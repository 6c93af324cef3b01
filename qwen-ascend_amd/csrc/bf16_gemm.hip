// Dense bf16 GEMM on MFMA for the shared expert and router projections of
// the prefill MoE block (fnx/engine.py:1786-1802 at more than four rows):
//
//   y[m, n] = bf16( sum_k a[m, k] * W[n, k] )   (F.linear, fp32 accumulation)
//
// a: bf16 rows of K (row m at a + m*lda), W: bf16 [N, K] row-major (the
// reference's Raw container), y: bf16 rows (row m at y + m*ldy).
//
// Tiles of 256 x 128, 128 x 128 or 64 x 64 outputs (the largest that still
// gives every CU a workgroup) per workgroup of 4 waves (2 x 2;
// v_mfma_f32_16x16x32_bf16 tiles of 16 x 16). K runs in 32-wide chunks
// staged through LDS in two buffers (64-wide chunks measured slower: the
// LDS they need leaves one workgroup per CU): while the waves multiply
// chunk c, the next chunk's 16-byte pieces of a and W are already in
// registers and land in the other buffer. Both operands keep K contiguous, so a lane's MFMA fragment (8 consecutive k of one row of a or
// of W) is one 16-byte LDS read; rows are padded by 8 elements so the 16
// rows a fragment read touches fall in different banks. Workgroups that share
// rows of a run on one XCD. Products of two bf16 are exact in fp32, so the
// result is the rounding of an fp32 accumulation of exact terms.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;

constexpr int kThreads = 256;
constexpr int BK = 32;    // k per MFMA step; K must be a multiple

// Block tile BM x BN, four waves in 2 x 2, each (BM/2) x (BN/2): TI x TJ MFMA
// tiles of 16 x 16 with TI = BM/32, TJ = BN/32; KC k per staged chunk (one
// or two MFMA steps), LDS rows of KC + 8 elements.
template <int BM, int BN, int KC>
__global__ __launch_bounds__(kThreads, 2) void bf16_gemm_kernel(const uint16_t* __restrict__ a, long lda,
                                                                const uint16_t* __restrict__ w,
                                                                uint16_t* __restrict__ y, long ldy, int M, int K,
                                                                int N) {
  constexpr int TI = BM / 32, TJ = BN / 32;
  constexpr int kPad = KC + 8;
  constexpr int PR = KC / 8;                  // 16-byte pieces per row and chunk
  constexpr int RPP = kThreads / PR;          // rows covered by one pass of the threads
  constexpr int AP = BM / RPP, BP = BN / RPP;  // 16-byte pieces per thread and chunk
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][BM * kPad];
  __shared__ __attribute__((aligned(16))) uint16_t sb[2][BN * kPad];
  const int ntn = (N + BN - 1) / BN;
  const int ntiles = ((M + BM - 1) / BM) * ntn;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  if (tile >= ntiles) return;
  const int m0 = (tile / ntn) * BM, n0 = (tile % ntn) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int i16 = lane & 15, kb = lane >> 4;

  // global pieces of a chunk: thread t copies 16-byte piece t % PR of rows
  // t / PR + RPP h (rows past the end re-read the last one)
  const int prow = tid / PR, pk = (tid % PR) * 8;
  const uint16_t* ap[AP];
  const uint16_t* wp[BP];
#pragma unroll
  for (int h = 0; h < AP; ++h) ap[h] = a + (size_t)min(m0 + prow + RPP * h, M - 1) * lda + pk;
#pragma unroll
  for (int h = 0; h < BP; ++h) wp[h] = w + (size_t)min(n0 + prow + RPP * h, N - 1) * K + pk;
  uint4 ra[AP], rb[BP];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int h = 0; h < AP; ++h) ra[h] = *reinterpret_cast<const uint4*>(ap[h] + k0);
#pragma unroll
    for (int h = 0; h < BP; ++h) rb[h] = *reinterpret_cast<const uint4*>(wp[h] + k0);
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int h = 0; h < AP; ++h) *reinterpret_cast<uint4*>(&sa[buf][(prow + RPP * h) * kPad + pk]) = ra[h];
#pragma unroll
    for (int h = 0; h < BP; ++h) *reinterpret_cast<uint4*>(&sb[buf][(prow + RPP * h) * kPad + pk]) = rb[h];
  };

  f32x4_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nch = K / KC;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    if (c + 1 < nch) fetch((c + 1) * KC);
#pragma unroll
    for (int st = 0; st < KC / BK; ++st) {
      bf16x8_v bf[TJ];
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        bf[j] = *reinterpret_cast<const bf16x8_v*>(&sb[buf][(wn * (BN / 2) + j * 16 + i16) * kPad + st * BK + kb * 8]);
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const bf16x8_v af =
            *reinterpret_cast<const bf16x8_v*>(&sa[buf][(wm * (BM / 2) + i * 16 + i16) * kPad + st * BK + kb * 8]);
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    if (c + 1 < nch) {
      stash(buf ^ 1);
      __syncthreads();
    }
  }

  // lane holds column i16 of tile (i, j) for rows 4*kb + r
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + wn * (BN / 2) + j * 16 + i16;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * (BM / 2) + i * 16 + 4 * kb + r;
        if (m < M) y[(size_t)m * ldy + n] = (uint16_t)f32_to_bf16(acc[i][j][r]);
      }
    }
}

}  // namespace

extern "C" {

int qmoe_bf16_gemm(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N, void* stream) {
  if (M < 1 || N < 1 || K < BK || (K % BK) || ldx < K || (ldx % 8) || ldy < N ||
      ((uintptr_t)x & 15) || ((uintptr_t)w & 15))
    return QMOE_EINVAL;
  auto launch = [&](auto kern, int bm, int bn) {
    const long tiles = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const long blocks = (tiles + 7) / 8 * 8;  // whole XCD rounds (extra blocks exit)
    if (blocks > 0x7fffffffL) return (int)QMOE_EINVAL;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                       ldx, (const uint16_t*)w, (uint16_t*)y, ldy, M, K, N);
    return (int)hipGetLastError();
  };
  // the largest tile that still gives every CU a workgroup: 256 x 128 (waves
  // of 128 x 64, the fewest LDS reads per MFMA), 128 x 128, else 64 x 64
  auto tiles = [&](long bm, long bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (tiles(256, 128) >= 256) return launch(bf16_gemm_kernel<256, 128, 32>, 256, 128);
  if (tiles(128, 128) >= 256) return launch(bf16_gemm_kernel<128, 128, 32>, 128, 128);
  return launch(bf16_gemm_kernel<64, 64, 32>, 64, 64);
}

}  // extern "C"
