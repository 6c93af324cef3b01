// W8A16 per-group GEMM: the int8 form of npu_weight_quant_batchmatmul used
// by the reference's dense projections (DenseW8, fnx/engine.py:297-384).
//
//   y[m, n] = bf16( sum_k x[m, k] * q[k, n] * S[k / gs, n] ),  fp32 accumulation
//
// q int8 [K, N] (row k holds the N columns), S bf16 [K/gs, N], x bf16 [M, K].
//
// M <= 4: split-K GEMV. A workgroup owns 256 columns (16 chunks of 16 bytes)
// and a K-slice of 16 L rows: thread (row-lane r = tid/16, chunk tid%16)
// loads its L rows of 16 columns at once (L = 4, 8 or 16, the most that
// keeps >= 512 workgroups in the grid and a run inside one scale group). A byte is read as offset binary u = q + 128
// (one xor per word) and converted by v_cvt_f32_ubyte; x * u is exact in
// fp32, and the accumulator starts at -128 * sum(x) so it ends at
// sum(x * q). A thread's 4 rows lie in one scale group, so it applies S once.
// Row-lanes are summed in LDS in row-lane order, the K-slices by the last
// workgroup to arrive, in slice order: deterministic run to run.
//
// M > 4: bf16 MFMA (16x16x32) on 64 x 64 output tiles. int8 values are exact
// in bf16, so the MFMA sums x * q exactly per product with fp32
// accumulation; after each scale group the group's partial sums are scaled by
// S[g, n] and added to the output accumulators.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunks = 16;                  // 16-byte chunks per tile row (256 columns)
constexpr int kTileCols = kChunks * 16;      // 256
constexpr int kRowLanes = kThreads / kChunks;  // 16
constexpr int kMaxL = 16;                    // largest rows per thread
constexpr int kRedStride = 17;               // LDS floats per (row-lane, chunk): 16 + 1 pad

template <int MR, int kL>
__global__ __launch_bounds__(kThreads) void w8a16_gemv_kernel(const uint16_t* __restrict__ x,
                                                              const int8_t* __restrict__ w,
                                                              const uint16_t* __restrict__ s,
                                                              uint16_t* __restrict__ y, int M, int K, int N, int gs,
                                                              float* __restrict__ part, int* __restrict__ counters) {
  __shared__ float red[kRowLanes * kChunks * kRedStride];
  __shared__ float res[MR][kTileCols];
  const int tile = blockIdx.x, slice = blockIdx.y, nslices = gridDim.y;
  const int tid = threadIdx.x;
  const int cc = tid % kChunks, r = tid / kChunks;
  const int col0 = tile * kTileCols + cc * 16;
  constexpr int kSlice = kRowLanes * kL;
  const int kr = slice * kSlice + r * kL;
  const bool active = col0 < N && kr < K;

  float acc[MR][16];
  if (active) {
    uint4 wv[kL];
#pragma unroll
    for (int i = 0; i < kL; ++i) wv[i] = *reinterpret_cast<const uint4*>(w + (size_t)(kr + i) * N + col0);
    const uint4* sp = reinterpret_cast<const uint4*>(s + (size_t)(kr / gs) * N + col0);
    const uint4 s0 = sp[0], s1 = sp[1];
    float xv[MR][kL], sx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      sx[m] = 0.f;
#pragma unroll
      for (int i = 0; i < kL; ++i) {
        xv[m][i] = m < M ? bf16_to_f32(x[(size_t)m * K + kr + i]) : 0.f;
        sx[m] += xv[m][i];
      }
#pragma unroll
      for (int c = 0; c < 16; ++c) acc[m][c] = -128.f * sx[m];
    }
#pragma unroll
    for (int i = 0; i < kL; ++i) {
      const uint32_t wd[4] = {wv[i].x ^ 0x80808080u, wv[i].y ^ 0x80808080u, wv[i].z ^ 0x80808080u,
                              wv[i].w ^ 0x80808080u};
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float u = (float)((wd[c >> 2] >> (8 * (c & 3))) & 0xffu);
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m][c] = __builtin_fmaf(xv[m][i], u, acc[m][c]);
      }
    }
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const float sc = bf16_to_f32((c & 1) ? (sw[c >> 1] >> 16) : (sw[c >> 1] & 0xffffu));
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m][c] *= sc;
    }
  } else {
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < 16; ++c) acc[m][c] = 0.f;
  }

  // row-lane sums in LDS, one x row at a time; column tid of the tile
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float* dst = red + (r * kChunks + cc) * kRedStride;
#pragma unroll
    for (int c = 0; c < 16; ++c) dst[c] = acc[m][c];
    __syncthreads();
    const float* src = red + (tid / 16) * kRedStride + (tid & 15);
    float sum = 0.f;
#pragma unroll
    for (int rr = 0; rr < kRowLanes; ++rr) sum += src[rr * kChunks * kRedStride];
    res[m][tid] = sum;
    __syncthreads();
  }

  const int col = tile * kTileCols + tid;
  if (nslices == 1) {
    if (col < N)
      for (int m = 0; m < M; ++m) y[(size_t)m * N + col] = (uint16_t)f32_to_bf16(res[m][tid]);
    return;
  }
  float* mypart = part + (size_t)slice * MR * N;
  if (col < N)
    for (int m = 0; m < M; ++m) store_agent(&mypart[(size_t)m * N + col], res[m][tid]);
  if (!arrive_last(counters + tile, nslices)) return;
  if (col >= N) return;
  for (int m = 0; m < M; ++m) {
    const float sum = sum_agent_ordered(&part[(size_t)m * N + col], (size_t)MR * N, nslices);
    y[(size_t)m * N + col] = (uint16_t)f32_to_bf16(sum);
  }
}

// ---------------------------------------------------------------- M > 4: MFMA

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

constexpr int kBM = 64, kBN = 64, kBK = 32;
constexpr int kLdsK = kBK + 8;  // bf16 per LDS row (16 bytes of pad against bank conflicts)

__global__ __launch_bounds__(kThreads) void w8a16_mfma_kernel(const uint16_t* __restrict__ x,
                                                              const int8_t* __restrict__ w,
                                                              const uint16_t* __restrict__ s,
                                                              uint16_t* __restrict__ y, int M, int K, int N, int gs) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kBM * kLdsK];  // [row][k]
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN * kLdsK];  // [col][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int wr = wave >> 1, wc = wave & 1;  // 32 x 32 quadrant of the wave
  f32x4_v acc[2][2], accg[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = accg[a][b] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  const int steps_per_group = gs / kBK;
  for (int k0 = 0, step = 0; k0 < K; k0 += kBK, ++step) {
    // A: 64 rows x 32 k (thread: row tid/4, 8 k at 8 (tid%4))
    {
      const int row = tid >> 2, kc = (tid & 3) * 8;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (m0 + row < M) v = *reinterpret_cast<const uint4*>(x + (size_t)(m0 + row) * K + k0 + kc);
      *reinterpret_cast<uint4*>(As + row * kLdsK + kc) = v;
    }
    // B: 32 k x 64 columns of int8 (threads 0..127: k tid/4, 16 columns at 16 (tid%4)),
    // written transposed as bf16 [col][k]
    if (tid < 128) {
      const int kk = tid >> 2, nc = (tid & 3) * 16;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (n0 + nc < N) v = *reinterpret_cast<const uint4*>(w + (size_t)(k0 + kk) * N + n0 + nc);
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const int q = (int)(int8_t)((wd[c >> 2] >> (8 * (c & 3))) & 0xffu);
        Bs[(nc + c) * kLdsK + kk] = (uint16_t)(__float_as_uint((float)q) >> 16);  // exact
      }
    }
    __syncthreads();
    const int kb = (lane >> 4) * 8;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const bf16x8_v af = *reinterpret_cast<const bf16x8_v*>(As + (wr * 32 + a * 16 + (lane & 15)) * kLdsK + kb);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const bf16x8_v bf = *reinterpret_cast<const bf16x8_v*>(Bs + (wc * 32 + b * 16 + (lane & 15)) * kLdsK + kb);
        accg[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, accg[a][b], 0, 0, 0);
      }
    }
    __syncthreads();
    if ((step + 1) % steps_per_group == 0) {
      // end of scale group g: acc += S[g, col] * group sums (lane holds column lane%16)
      const int g = k0 / gs;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int col = n0 + wc * 32 + b * 16 + (lane & 15);
        const float sc = col < N ? bf16_to_f32(s[(size_t)g * N + col]) : 0.f;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[a][b][i] = __builtin_fmaf(accg[a][b][i], sc, acc[a][b][i]);
          accg[a][b] = f32x4_v{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
  // D layout: lane holds rows 4 (lane/16) .. +3 of column lane%16
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int col = n0 + wc * 32 + b * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + wr * 32 + a * 16 + (lane >> 4) * 4 + i;
        if (row < M && col < N) y[(size_t)row * N + col] = (uint16_t)f32_to_bf16(acc[a][b][i]);
      }
    }
}

}  // namespace

extern "C" {

// Rows per thread for a shape: the largest L in {16, 8, 4} (up to kMaxL)
// that divides gs and still leaves >= 512 workgroups (or is 4).
static int w8_rows_per_thread(int K, int N, int gs) {
  for (int L = kMaxL; L > 4; L >>= 1)
    if (gs % L == 0 && (long)host_ceil_div(N, kTileCols) * host_ceil_div(K, kRowLanes * L) >= 512) return L;
  return 4;
}

size_t qmoe_w8a16_gemv_workspace(int M, int K, int N) {
  (void)M;
  return (size_t)host_ceil_div(K, kRowLanes * 4) * 4 * (size_t)N * sizeof(float);
}

int qmoe_w8a16_gemv_counters(int N) { return host_ceil_div(N, kTileCols); }

int qmoe_w8a16_gemv(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int group_size,
                    void* workspace, size_t workspace_bytes, void* counters, void* stream) {
  if (M < 1 || M > 4 || K < 4 || (K % 4) || N < 16 || (N % 16) || group_size < 4 || (group_size % 4) ||
      (K % group_size) || host_ceil_div(N, kTileCols) >= QMOE_DECODE_MAILBOX_BASE - 1)
    return QMOE_EINVAL;
  const int L = w8_rows_per_thread(K, N, group_size);
  const int nslices = host_ceil_div(K, kRowLanes * L);
  if (nslices > 1 && workspace_bytes < qmoe_w8a16_gemv_workspace(M, K, N)) return QMOE_EWORKSPACE;
  dim3 grid(host_ceil_div(N, kTileCols), nslices);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x, (const int8_t*)w,
                       (const uint16_t*)scale, (uint16_t*)y, M, K, N, group_size, (float*)workspace,
                       (int*)counters);
  };
#define QMOE_W8_L(L_)                                                   \
  if (L == L_) {                                                        \
    if (M == 1) go(w8a16_gemv_kernel<1, L_>);                           \
    else if (M == 2) go(w8a16_gemv_kernel<2, L_>);                      \
    else go(w8a16_gemv_kernel<4, L_>);                                  \
    return (int)hipGetLastError();                                      \
  }
  QMOE_W8_L(16) QMOE_W8_L(8) QMOE_W8_L(4)
#undef QMOE_W8_L
  return QMOE_EINVAL;
}

int qmoe_w8a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                         int group_size, void* stream) {
  if (M < 1 || K < kBK || (K % kBK) || N < 16 || (N % 16) || group_size < kBK || (group_size % kBK) ||
      (K % group_size) || host_ceil_div(M, kBM) > 65535)
    return QMOE_EINVAL;
  dim3 grid(host_ceil_div(N, kBN), host_ceil_div(M, kBM));
  hipLaunchKernelGGL(w8a16_mfma_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                     (const int8_t*)w, (const uint16_t*)scale, (uint16_t*)y, M, K, N, group_size);
  return (int)hipGetLastError();
}

}  // extern "C"
