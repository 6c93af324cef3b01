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
// M > 4: bf16 MFMA (16x16x32) on 64- or 128-row, 64-column output tiles,
// the operands streaming through an LDS ring of chunks. int8 values are exact in bf16, so the MFMA sums
// x * q exactly per product with fp32 accumulation; after each scale group
// the group's partial sums are scaled by S[g, n] and added to the output
// accumulators.
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
    for (int i = 0; i < kL; ++i) wv[i] = load_nt16(w + (size_t)(kr + i) * N + col0);
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
//
// bf16 MFMA 16x16x32 on BM x BN output tiles per workgroup of 4 waves (2 x 2,
// each (BM/2) x (BN/2): TI x TJ MFMA tiles). K runs in KC-wide chunks (one
// or two MFMA steps) that stream into a ring of RING LDS slots by
// buffer-resource global->LDS DMA, RING - 1 chunks ahead: the x rows (16-byte
// pieces of a row stored XOR-swizzled by row, so the 16 rows a fragment
// read touches fall in different banks), the raw int8 weight rows [KC][BN]
// (row k in row slot k ^ ((k / 4) % (256 / BN)), so the four rows a
// conversion read touches fall in different banks) and the bf16 scale row of
// the chunk's group. One chunk ahead of the MFMAs
// every thread converts a 4 k x CPT block of that chunk's weights to bf16
// (exact: |q| <= 128 has at most 8 significant bits) into one of two
// transposed buffers [column][k] (rows padded by 4 elements), so a lane's B
// fragment (8 consecutive k of one column) is two 8-byte reads; one barrier
// per chunk orders it all. Every LDS layout here keeps the lanes of one
// access in different banks. The MFMAs of one scale
// group sum into group accumulators; at the group's end those are scaled by
// S[g, n] with one fp32 fma into the output accumulators and cleared.

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;                     // k per MFMA step

QMOE_DEV uint32_t i8_to_bf16_bits(uint32_t word, int byte) {
  return __float_as_uint((float)(int)(int8_t)(word >> (8 * byte))) >> 16;
}

// s_waitcnt with vmcnt <= N and lgkmcnt == 0 (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4] left at 7).
template <int N>
QMOE_DEV void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4));
}

// An 8-byte LDS write the compiler does not track. It cannot tell which LDS
// bytes an in-flight global->LDS DMA writes, so before an ordinary LDS store
// it would wait for every outstanding DMA (the chunks prefetched ahead too);
// used only for the converted weights, which no DMA touches.
QMOE_DEV void lds_write8_untracked(void* p, uint32_t lo, uint32_t hi) {
  const unsigned a = (unsigned)(size_t)(__attribute__((address_space(3))) char*)p;
  asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(make_uint2(lo, hi)) : "memory");
}

// The weight fragments of a chunk's two MFMA steps (two per step, 16 columns
// apart), each read from the converted rows as two 8-byte halves, in one
// block that waits for its own reads. An ordinary LDS load here would make
// the compiler wait for every global->LDS DMA in flight (the chunk just issued
// included), since it cannot tell which LDS bytes a DMA writes; no DMA writes
// the converted buffers.
QMOE_DEV void lds_read_frags4(const void* p0, const void* p1, const void* p2, const void* p3, uint4& f0, uint4& f1,
                              uint4& f2, uint4& f3) {
  auto a = [](const void* p) { return (unsigned)(size_t)(__attribute__((address_space(3))) const char*)p; };
  asm volatile(
      "ds_read2_b64 %0, %4 offset1:1\n\t"
      "ds_read2_b64 %1, %5 offset1:1\n\t"
      "ds_read2_b64 %2, %6 offset1:1\n\t"
      "ds_read2_b64 %3, %7 offset1:1\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(f0), "=&v"(f1), "=&v"(f2), "=&v"(f3)
      : "v"(a(p0)), "v"(a(p1)), "v"(a(p2)), "v"(a(p3))
      : "memory");
}

template <int V>
struct W8C {
  static constexpr int value = V;
};

template <int BM_, int BN_, int KC_, int RING_>
struct W8Tile {
  static constexpr int BM = BM_, BN = BN_, KC = KC_, RING = RING_;
  static constexpr int TI = BM / 32, TJ = BN / 32;
  static constexpr int NS = KC / kBK;                   // MFMA steps per chunk
  static constexpr int PPR = KC / 8;                    // 16-byte pieces per x row and chunk
  static constexpr int A_BYTES = BM * 2 * KC;           // x rows of one chunk
  static constexpr int B_BYTES = KC * BN;               // raw int8 weight rows of one chunk
  static constexpr int S_BYTES = BN * 2;                // bf16 scale row of the chunk's group
  static constexpr int SLOT = A_BYTES + B_BYTES + S_BYTES;
  static constexpr int AQ = A_BYTES / 1024 / 4;         // A DMA instructions per wave and chunk
  static constexpr int BQ = B_BYTES / 1024;             // B DMA instructions per chunk (1 KB each)
  static constexpr int BQW = (BQ + 3) / 4;              // ... per wave (waves past BQ repeat the last one)
  static constexpr int IPC = AQ + BQW + 1;              // DMA instructions per wave and chunk (1: scales)
  static constexpr int KG = KC / 4;                     // converting threads' k-row groups of 4
  static constexpr int CG = kThreads / KG;              // ... and their column groups
  static constexpr int CPT = BN / CG;                   // weight columns per converting thread
  static constexpr int RPS = BN >= 256 ? 1 : 256 / BN;  // raw weight rows per sweep of the 64 LDS banks
  static constexpr int LDK = KC + 4;                    // bf16 per row of the converted weights (8-byte aligned)
  static constexpr int CONV = 2 * BN * LDK * 2;         // two converted weight buffers
  static constexpr int LDS = RING * SLOT + CONV;
  static_assert(A_BYTES % 4096 == 0 && (CPT == 2 || CPT == 4 || CPT == 8), "tile shape");
};

template <class T>
__global__ __launch_bounds__(kThreads) void w8a16_mfma_kernel(const uint16_t* __restrict__ x,
                                                              const int8_t* __restrict__ w,
                                                              const uint16_t* __restrict__ s,
                                                              uint16_t* __restrict__ y, int M, int K, int N, int gs) {
  constexpr int BM = T::BM, BN = T::BN, KC = T::KC, RING = T::RING;
  constexpr int TI = T::TI, TJ = T::TJ, CPT = T::CPT, PPR = T::PPR, LDK = T::LDK;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  uint16_t* sbc = reinterpret_cast<uint16_t*>(lds + RING * T::SLOT);  // [2][BN][LDK]
  const int ntn = (N + BN - 1) / BN;
  const int ntiles = ((M + BM - 1) / BM) * ntn;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  if (tile >= ntiles) return;
  const int m0 = (tile / ntn) * BM, n0 = (tile % ntn) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave >> 1, wn = wave & 1;
  const int i16 = lane & 15, kb = lane >> 4;
  // piece swizzle of x row r: the 16 rows of a fragment read spread over the banks
  auto swz = [](int r) { return PPR == 4 ? ((r >> 2) & 3) : (r & 7); };

  // ---- DMA sources. A instruction q of wave w: rows (64 / PPR) (4q + w) +
  // lane / PPR, LDS piece lane % PPR of the row holding k-piece
  // (lane % PPR) ^ swz(row). B instruction b: 1 KB of the raw [KC][BN] chunk,
  // lane l at byte 16 l. Scales: lane l < BN / 32 of wave w fetches 8 columns
  // at w BN / 4 + 8 l of the chunk's group row. Buffer resources bound every
  // access to its tensor; the per-lane offsets are fixed and a wave-uniform
  // offset advances per chunk.
  constexpr int kRsrcWord3 = 0x00020000;
  const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, M * K * 2, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, K * N, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_s =
      __builtin_amdgcn_make_buffer_rsrc((void*)s, (short)0, (K / gs) * N * 2, kRsrcWord3);
  uint32_t aoff[T::AQ], boff[T::BQW];
#pragma unroll
  for (int q = 0; q < T::AQ; ++q) {
    const int r = (64 / PPR) * (4 * q + wave) + lane / PPR;
    const int piece = (lane % PPR) ^ swz(r);
    aoff[q] = 2u * ((uint32_t)min(m0 + r, M - 1) * (uint32_t)K + 8u * (uint32_t)piece);
  }
  // raw weight row k sits in LDS row slot k ^ ((k / 4) % RPS) (an involution):
  // the four rows a converting thread reads at once are then in different banks
  auto row_slot = [](int k) { return k ^ ((k >> 2) & (T::RPS - 1)); };
#pragma unroll
  for (int q = 0; q < T::BQW; ++q) {
    const int b = min(4 * q + wave, T::BQ - 1);
    const int byte = 1024 * b + 16 * lane;
    boff[q] = (uint32_t)row_slot(byte / BN) * (uint32_t)N + (uint32_t)(n0 + byte % BN);
  }
  const uint32_t soff = 2u * (uint32_t)(n0 + wave * (BN / 4) + 8 * (lane & (BN / 32 - 1)));
  auto issue_chunk = [&](int c, int slot) {
    unsigned char* base = lds + slot * T::SLOT;
    const int k0 = c * KC;
#pragma unroll
    for (int q = 0; q < T::AQ; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (__attribute__((address_space(3))) void*)(base + (4 * q + wave_u) * 1024),
                                               16, (int)aoff[q], k0 * 2, 0, 0);
#pragma unroll
    for (int q = 0; q < T::BQW; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc_b, (__attribute__((address_space(3))) void*)(base + T::A_BYTES + min(4 * q + wave_u, T::BQ - 1) * 1024), 16,
          (int)boff[q], k0 * N, 0, 0);
    if (lane < BN / 32)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_s,
                                               (__attribute__((address_space(3))) void*)(base + T::A_BYTES + T::B_BYTES + wave_u * (BN / 2)),
                                               16, (int)soff, (k0 / gs) * N * 2, 0, 0);
  };
  // ---- conversion of chunk c's raw weights into converted buffer c % 2:
  // thread t takes k rows 4 (t / CG) .. + 3 of columns CPT (t % CG) .. + CPT - 1
  // (row 4 kg + r from its slot)
  const int kg = tid / T::CG, cg = tid % T::CG;
  int rawoff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) rawoff[r] = row_slot(4 * kg + r) * BN + CPT * cg;
  constexpr int NW = (CPT + 3) / 4;
  // the raw weight words a thread converts (convert_load), then their bf16
  // rows written to converted buffer buf (convert_store)
  auto convert_load = [&](int slot, uint32_t (&rw)[4][NW]) {
    const unsigned char* raw = lds + slot * T::SLOT + T::A_BYTES;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const unsigned char* p = raw + rawoff[r];
      if constexpr (CPT == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        rw[r][0] = v.x;
        rw[r][1] = v.y;
      } else if constexpr (CPT == 4) {
        rw[r][0] = *reinterpret_cast<const uint32_t*>(p);
      } else {
        rw[r][0] = (uint32_t)*reinterpret_cast<const uint16_t*>(p);
      }
    }
  };
  auto convert_store = [&](int buf, const uint32_t (&rw)[4][NW]) {
    uint16_t* dst = sbc + buf * BN * LDK + (CPT * cg) * LDK + 4 * kg;
#pragma unroll
    for (int cc = 0; cc < CPT; ++cc) {
      const int wd = cc >> 2, by = cc & 3;
      const uint32_t lo = i8_to_bf16_bits(rw[0][wd], by) | (i8_to_bf16_bits(rw[1][wd], by) << 16);
      const uint32_t hi = i8_to_bf16_bits(rw[2][wd], by) | (i8_to_bf16_bits(rw[3][wd], by) << 16);
      lds_write8_untracked(dst + cc * LDK, lo, hi);
    }
  };

  f32x4_v acc[TI][TJ], accg[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = accg[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  int col[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j) col[j] = n0 + wn * (BN / 2) + j * 16 + i16;
  // A fragment rows of this lane (tile i: row wm BM/2 + 16 i + i16)
  int arow[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) arow[i] = wm * (BM / 2) + 16 * i + i16;

  const int nch = K / KC, cpg = gs / KC;
  // ---- prologue: chunks 0 .. RING - 2 in flight, chunk 0 converted
#pragma unroll
  for (int c = 0; c < RING - 1; ++c)
    if (c < nch) issue_chunk(c, c);
  if (nch >= RING - 1) wait_vm_lgkm0<(RING - 2) * T::IPC>();
  else __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  {
    uint32_t rw[4][NW];
    convert_load(0, rw);
    convert_store(0, rw);
  }

  // one chunk: ring slot SL = c % RING and converted buffer BU = c % 2 are
  // compile-time constants (the loop below is unrolled over lcm(RING, 2)
  // chunks), so every LDS address is an immediate offset; FIRST: c starts a
  // scale group, whose first MFMAs take a zero accumulator instead of the
  // group sums being cleared after each group
  auto chunk = [&](auto sl_c, auto bu_c, auto first_c, int c) {
    constexpr int SL = decltype(sl_c)::value, BU = decltype(bu_c)::value;
    constexpr bool FIRST = decltype(first_c)::value != 0;
    // chunk c + 1 has landed once only the later chunks in flight may be
    // pending; this chunk's converted rows (LDS stores) are complete
    if (c + 1 < nch) {
      if (c + RING - 2 < nch) wait_vm_lgkm0<(RING - 3) * T::IPC>();
      else __builtin_amdgcn_s_waitcnt(0);
    } else {
      wait_vm_lgkm0<63>();
    }
    // every wave is past chunk c - 1: its ring slot and converted buffer are
    // free. No fence: it would also wait for the chunks prefetched ahead.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + RING - 1 < nch) issue_chunk(c + RING - 1, (SL + RING - 1) % RING);
    // Every LDS read of the chunk goes out together: the raw words of chunk
    // c + 1 to convert, both steps' weight and activation fragments and, at
    // the end of a scale group, the group's scale row. Step 0's MFMAs then run
    // beside the conversion, whose stores precede step 1.
    const bool convert_next = c + 1 < nch;
    const bool group_end = (c + 1) % cpg == 0;
    uint32_t rw[4][NW];
    if (convert_next) convert_load((SL + 1) % RING, rw);
    const unsigned char* as = lds + SL * T::SLOT;
    bf16x8_v bf[T::NS][TJ], af[T::NS][TI];
#pragma unroll
    for (int st = 0; st < T::NS; ++st) {
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int r = arow[i];
        af[st][i] = *reinterpret_cast<const bf16x8_v*>(as + r * (2 * KC) + (((4 * st + kb) ^ swz(r)) << 4));
      }
    }
    {
      // weight fragments of both steps (converted rows are 8-byte aligned)
      static_assert(TJ == 2, "two weight fragments per wave and step");
      const uint16_t* bs = sbc + BU * BN * LDK + (wn * (BN / 2) + i16) * LDK + kb * 8;
      uint4 f[4];
      lds_read_frags4(bs, bs + 16 * LDK, bs + (T::NS - 1) * kBK, bs + 16 * LDK + (T::NS - 1) * kBK, f[0], f[1], f[2],
                      f[3]);
#pragma unroll
      for (int st = 0; st < T::NS; ++st)
#pragma unroll
        for (int j = 0; j < TJ; ++j) bf[st][j] = __builtin_bit_cast(bf16x8_v, f[(st ? 2 : 0) + j]);
    }
    float sc[TJ];
    if (group_end) {
      // the group's scale row came with this chunk
      const uint16_t* srow = reinterpret_cast<const uint16_t*>(as + T::A_BYTES + T::B_BYTES);
#pragma unroll
      for (int j = 0; j < TJ; ++j) sc[j] = col[j] < N ? bf16_to_f32(srow[wn * (BN / 2) + j * 16 + i16]) : 0.f;
    }
#pragma unroll
    for (int st = 0; st < T::NS; ++st) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          accg[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              af[st][i], bf[st][j], (FIRST && st == 0) ? f32x4_v{0.f, 0.f, 0.f, 0.f} : accg[i][j], 0, 0, 0);
      if (st == 0 && convert_next) convert_store(1 - BU, rw);
    }
    if (group_end) {
      // end of scale group: acc += S[g, col] * group sums
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(accg[i][j][r], sc[j], acc[i][j][r]);
    }
  };
  auto chunk_at = [&](auto sl_c, auto bu_c, int c) {
    if (c % cpg == 0) chunk(sl_c, bu_c, W8C<1>{}, c);
    else chunk(sl_c, bu_c, W8C<0>{}, c);
  };
  // the loop is unrolled over lcm(RING, 2) chunks
  constexpr int UN = RING % 2 == 0 ? RING : 2 * RING;
  auto unrolled = [&](auto self, auto j_c, int c) {
    constexpr int J = decltype(j_c)::value;
    if constexpr (J < UN) {
      if (c + J < nch) {
        chunk_at(W8C<J % RING>{}, W8C<J % 2>{}, c + J);
        self(self, W8C<J + 1>{}, c);
      }
    }
  };
  for (int c = 0; c < nch; c += UN) unrolled(unrolled, W8C<0>{}, c);
  // D layout: lane holds column i16 of tile (i, j) for rows 4 kb .. 4 kb + 3
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      if (col[j] >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * (BM / 2) + i * 16 + 4 * kb + r;
        if (row < M) y[(size_t)row * N + col[j]] = (uint16_t)f32_to_bf16(acc[i][j][r]);
      }
    }
}

template <class T>
int launch_w8_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int gs,
                   hipStream_t stream) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  if (dev < 0 || dev >= 64) return QMOE_EINVAL;
  static bool attr_set[64] = {};
  if (!attr_set[dev]) {
    err = hipFuncSetAttribute((const void*)w8a16_mfma_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, T::LDS);
    if (err != hipSuccess) return (int)err;
    attr_set[dev] = true;
  }
  const long tiles = (long)((M + T::BM - 1) / T::BM) * ((N + T::BN - 1) / T::BN);
  const long blocks = (tiles + 7) / 8 * 8;  // whole XCD rounds (extra blocks exit)
  if (blocks > 0x7fffffffL) return QMOE_EINVAL;
  hipLaunchKernelGGL(w8a16_mfma_kernel<T>, dim3((unsigned)blocks), dim3(kThreads), T::LDS, stream,
                     (const uint16_t*)x, (const int8_t*)w, (const uint16_t*)scale, (uint16_t*)y, M, K, N, gs);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

// Rows per thread for a shape: the largest L in {16, 8, 4} (up to kMaxL)
// that divides gs and still leaves >= 256 workgroups, one per CU (or is 4).
// With the weights read nontemporally the longer rows won: 2048 x 8192
// took 9.0 us with L = 16 (256 workgroups) against 9.9 with L = 8 (512).
static int w8_rows_per_thread(int K, int N, int gs) {
  for (int L = kMaxL; L > 4; L >>= 1)
    if (gs % L == 0 && (long)host_ceil_div(N, kTileCols) * host_ceil_div(K, kRowLanes * L) >= 256) return L;
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
      (K % group_size) || ((uintptr_t)x & 15) || ((uintptr_t)w & 15) ||
      (long)M * K * 2 >= 0x80000000L || (long)K * N >= 0x80000000L)
    return QMOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  // 128 x 64 tiles where they still give every CU a workgroup (64-k chunks
  // when the group size allows: twice the MFMA work per barrier), else 64 x 64
  const long tiles128 = (long)((M + 127) / 128) * ((N + 63) / 64);
  if (tiles128 >= 256 && group_size % 64 == 0 && K % 64 == 0)
    return launch_w8_mfma<W8Tile<128, 64, 64, 3>>(x, w, scale, y, M, K, N, group_size, st);
  if (tiles128 >= 256) return launch_w8_mfma<W8Tile<128, 64, 32, 4>>(x, w, scale, y, M, K, N, group_size, st);
  return launch_w8_mfma<W8Tile<64, 64, 32, 4>>(x, w, scale, y, M, K, N, group_size, st);
}

}  // extern "C"
