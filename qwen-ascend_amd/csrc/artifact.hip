// Artifact conversion on the GPU: the LQP expert layout (v2o, offset-binary
// int4 packed along K) to the int4pack W4A16 container (packed along N), and
// the LQP scale pair to the s8t / bf16 base / bf16 scale-cache tensors.
//
// v2o, uint8 [E, N, K/2] (tools/repack_v2.py:39-54): for every 128-wide K
// segment s of row n, byte 64s+j holds W[n, 128s+j] + 8 in its low nibble and
// W[n, 128s+64+j] + 8 in its high nibble.
// int4pack, int32 (tools/repack_w4a16.py:58-76): word c of row k holds
// W[k, 8c+j] in nibble j (low first), two's complement. Expert-major
// [E, K, N/8] (tools/repack_w4_em.py:16) or K-major [K, E, N/8].
//
// The conversion is a nibble transpose (K-contiguous rows to N-contiguous
// rows): a workgroup takes 256 rows n x one 128-wide K segment of one expert
// (16 KiB of v2o, one 64-byte piece per row, loaded as 16-byte vectors), puts
// it in LDS, and writes the 128 int4pack rows of those 256 columns (128 bytes
// each, whole lines). Offset binary becomes two's complement by flipping
// each nibble's top bit.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTileN = 256;          // rows n per workgroup
constexpr int kSeg = 128;            // K per v2o segment
constexpr int kRowBytes = kSeg / 2;  // v2o bytes of one row in one segment

// SPW v2o segments per workgroup (1, or 2 when K allows: 128-byte row pieces
// in, 16-byte stores out).
template <int SPW>
__global__ __launch_bounds__(kThreads) void lqp_to_int4pack_kernel(const uint8_t* __restrict__ v2o,
                                                                   uint32_t* __restrict__ w4, int E, int N, int K,
                                                                   int expert_major) {
  constexpr int kPiece = kRowBytes * SPW;  // v2o bytes of one row in the workgroup's segments
  constexpr int kLdsRow = kPiece + 4;      // padded LDS row (bytes)
  constexpr int kPieces = kPiece / 16;     // 16-byte loads per row
  constexpr int kCg = 16 / SPW;            // column groups of the store phase
  constexpr int kCols = kTileN / kCg;      // columns per thread (16 SPW)
  constexpr int kWords = kCols / 8;        // output words per thread and k row (2 SPW)
  __shared__ uint8_t tile[kTileN * kLdsRow];
  const int n0 = blockIdx.x * kTileN;
  const int s0 = blockIdx.y * SPW;  // first K segment
  const int e = blockIdx.z;
  const int tid = threadIdx.x;
  const size_t row_bytes = (size_t)K / 2;
  // load: thread t takes 16-byte pieces (row n0 + t / kPieces + (256 / kPieces) i, piece t % kPieces)
#pragma unroll
  for (int i = 0; i < kPieces; ++i) {
    const int r = tid / kPieces + (kThreads / kPieces) * i, p = tid % kPieces;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (n0 + r < N)
      v = load_nt16(v2o + ((size_t)e * N + n0 + r) * row_bytes + (size_t)s0 * kRowBytes + 16 * p);  // read once
    uint32_t* d = reinterpret_cast<uint32_t*>(tile + r * kLdsRow + 16 * p);
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
  }
  __syncthreads();
  // store: thread t = (column group cg = t % kCg, byte group jg = t / kCg)
  // reads one 32-bit word per column of its kCols columns n0 + kCols cg ..:
  // bytes 4 jg .. 4 jg + 3 of the row piece, in segment s0 + (4 jg) / 64,
  // whose low nibbles are k = 4 jg % 64 + q and high nibbles k = 64 + 4 jg % 64
  // + q (q = 0..3) of that segment. A 4x4 byte transpose per four columns
  // (v_perm) and a nibble compress give the kWords int4pack words of each of
  // those 8 k rows, stored as one piece per row: a wave's store covers
  // 64 / kCg rows, 128 bytes each.
  const int cg = tid % kCg, jg = tid / kCg;
  const int nw = N / 8;
  uint32_t rw[kCols];
#pragma unroll
  for (int i = 0; i < kCols; ++i)
    rw[i] = *reinterpret_cast<const uint32_t*>(tile + (kCols * cg + i) * kLdsRow + 4 * jg);
  // nibbles at bit 8b (b = 0..3, low four bits of each byte) packed to bit 4b
  auto compress = [](uint32_t x) -> uint32_t {
    x = (x | (x >> 4)) & 0x00FF00FFu;
    return (x | (x >> 8)) & 0x0000FFFFu;
  };
  const int c0 = (n0 >> 3) + kWords * cg;  // first of the thread's output words
  const int kseg = (s0 + (4 * jg) / kRowBytes) * kSeg + (4 * jg) % kRowBytes;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // byte q of the column words, four columns per register (column order)
    uint32_t t4[kCols / 4];
#pragma unroll
    for (int g4 = 0; g4 < kCols / 4; ++g4) {
      const uint32_t sel = (uint32_t)q | ((uint32_t)(q + 4) << 8) | 0x0C0C0000u;  // byte q of a, of b
      const uint32_t lo = __builtin_amdgcn_perm(rw[4 * g4 + 1], rw[4 * g4], sel);
      const uint32_t hi = __builtin_amdgcn_perm(rw[4 * g4 + 3], rw[4 * g4 + 2], sel);
      t4[g4] = lo | (hi << 16);
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      // half 0: low nibbles, half 1: high nibbles (64 k further)
      const int k = kseg + 64 * half + q;
      uint32_t word[kWords];
#pragma unroll
      for (int w = 0; w < kWords; ++w) {
        const uint32_t a = half ? (t4[2 * w] >> 4) : t4[2 * w];
        const uint32_t b = half ? (t4[2 * w + 1] >> 4) : t4[2 * w + 1];
        word[w] = (compress(a & 0x0F0F0F0Fu) | (compress(b & 0x0F0F0F0Fu) << 16)) ^ 0x88888888u;  // offset binary -> two's complement
      }
      uint32_t* out_row = expert_major ? w4 + ((size_t)e * K + k) * nw : w4 + ((size_t)k * E + e) * nw;
      if (c0 + kWords <= nw && (nw % kWords) == 0) {  // whole, aligned piece
        if constexpr (kWords == 4)
          *reinterpret_cast<uint4*>(out_row + c0) = make_uint4(word[0], word[1], word[2], word[3]);
        else
          *reinterpret_cast<uint2*>(out_row + c0) = make_uint2(word[0], word[1]);
      } else {
#pragma unroll
        for (int w = 0; w < kWords; ++w)
          if (c0 + w < nw) out_row[c0 + w] = word[w];
      }
    }
  }
}

// s8 int8 [E, N, G], base fp16 [E, N] ->
//   s8t int8 [G, E, N] (tools/repack_w4a16.py:71), base bf16 [E, N] (:72),
//   scales bf16 [E, G, N] = bf16(float(s8) * base_bf16) (fnx/engine.py:653-659).
// One thread per (e, n) column, looping over its G groups.
__global__ __launch_bounds__(kThreads) void lqp_scales_kernel(const int8_t* __restrict__ s8,
                                                              const uint16_t* __restrict__ base_f16,
                                                              int8_t* __restrict__ s8t, uint16_t* __restrict__ base_bf,
                                                              uint16_t* __restrict__ scales, int E, int N, int G) {
  const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;  // e * N + n
  if (i >= (size_t)E * N) return;
  const int e = (int)(i / N), n = (int)(i % N);
  const float bf = round_bf16((float)__builtin_bit_cast(_Float16, base_f16[i]));
  if (base_bf != nullptr) base_bf[i] = (uint16_t)f32_to_bf16(bf);
  const int8_t* src = s8 + i * G;
  for (int g = 0; g < G; ++g) {
    const int8_t v = src[g];
    if (s8t != nullptr) s8t[((size_t)g * E + e) * N + n] = v;
    if (scales != nullptr) scales[((size_t)e * G + g) * N + n] = (uint16_t)f32_to_bf16((float)v * bf);
  }
}

// Scale cache of the W4A16 container (fnx/engine.py:653-659): scales[e, g, n]
// = bf16(bf16(s8t[g, e, n]) * base[e, n]). The int8 value is exact in bf16
// and the product of two bf16 is exact in fp32, so one rounding gives the
// bf16 multiply's result. One thread per (e, n) column walks its G groups.
__global__ __launch_bounds__(kThreads) void scale_cache_kernel(const int8_t* __restrict__ s8t,
                                                               const uint16_t* __restrict__ base,
                                                               uint16_t* __restrict__ scales, int G, int E, int N) {
  const size_t col = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (col >= (size_t)E * N) return;
  const size_t e = col / N, n = col % N;
  const float b = bf16_to_f32(base[col]);
  for (int g = 0; g < G; ++g)
    scales[(e * G + g) * N + n] = (uint16_t)f32_to_bf16((float)s8t[((size_t)g * E + e) * N + n] * b);
}

}  // namespace

extern "C" {

int qmoe_lqp_to_int4pack(const void* v2o, void* w4, int E, int N, int K, int expert_major, void* stream) {
  if (E < 1 || N < 8 || (N % 8) || K < kSeg || (K % kSeg) || E > 65535 || K / kSeg > 65535) return QMOE_EINVAL;
  if ((reinterpret_cast<uintptr_t>(v2o) & 15) || (reinterpret_cast<uintptr_t>(w4) & 15)) return QMOE_EINVAL;
  if (K % (2 * kSeg) == 0) {
    dim3 grid(host_ceil_div(N, kTileN), K / (2 * kSeg), E);
    hipLaunchKernelGGL(lqp_to_int4pack_kernel<2>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)v2o,
                       (uint32_t*)w4, E, N, K, expert_major);
  } else {
    dim3 grid(host_ceil_div(N, kTileN), K / kSeg, E);
    hipLaunchKernelGGL(lqp_to_int4pack_kernel<1>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)v2o,
                       (uint32_t*)w4, E, N, K, expert_major);
  }
  return (int)hipGetLastError();
}

int qmoe_lqp_scales(const void* s8, const void* base_fp16, void* s8t, void* base_bf16, void* scales, int E, int N,
                    int G, void* stream) {
  if (E < 1 || N < 1 || G < 1) return QMOE_EINVAL;
  const size_t cols = (size_t)E * N;
  hipLaunchKernelGGL(lqp_scales_kernel, dim3((unsigned)((cols + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const int8_t*)s8, (const uint16_t*)base_fp16, (int8_t*)s8t,
                     (uint16_t*)base_bf16, (uint16_t*)scales, E, N, G);
  return (int)hipGetLastError();
}

int qmoe_scale_cache(const void* s8t, const void* base_bf16, void* scales, int G, int E, int N, void* stream) {
  if (G < 1 || E < 1 || N < 1) return QMOE_EINVAL;
  const size_t cols = (size_t)E * N;
  hipLaunchKernelGGL(scale_cache_kernel, dim3((unsigned)((cols + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const int8_t*)s8t, (const uint16_t*)base_bf16, (uint16_t*)scales, G, E, N);
  return (int)hipGetLastError();
}

}  // extern "C"
