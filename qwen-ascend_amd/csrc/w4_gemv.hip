// W4A16 GEMV / skinny GEMM (M <= 4) over int4pack weights, and the fused
// one-to-four-token MoE decode block built on it.
//
// Weight layout (int4pack, the reference's container): int32 [K, N/8]; nibble
// j of word c in row k is W[k, 8c+j], two's complement, low nibble first.
// Scales: bf16 [G, N], G = K / gs, symmetric, no zero point.
//
// Work split. A workgroup (256 threads) owns a 256-column tile (8 chunks of
// 32 columns, one 16-byte load per row per chunk) and a K-slice of 32*L rows:
// thread (row-lane r = tid/8, chunk cc = tid%8) streams rows
// [k0 + r*L, k0 + r*L + L) of its chunk with 16-byte loads (8 threads cover
// 256 contiguous bytes of a row, so every wave load is fully coalesced).
//
// Arithmetic. Two rows k, k+1 of a chunk are unpacked together into bf16
// pairs (W[k,n], W[k+1,n]) encoded as 16 + u = q + 24 with u = q + 8 (nibble
// placed in the top mantissa bits, exponent of 16), and dotted with
// (x[k], x[k+1]) by v_dot2c_f32_bf16 into an fp32 accumulator that starts at
// -24 * sum_k x, so it ends at sum_k x*q. Every product is exact in fp32. A
// thread's L rows lie in one scale group, so it applies S[g, n] once per run.
// Per-column results of the 32 row-lanes are summed in LDS in row-lane
// order, then across K-slices in slice order by the last workgroup to finish
// the tile (an atomic arrival counter that the finisher resets to zero), so
// results are deterministic run to run and no second launch is needed.
#include "qmoe_common.h"
#include "qmoe.h"

#include <mutex>

namespace {

constexpr int kThreads = 256;
constexpr int kChunks = 8;                     // 32-column chunks per tile
constexpr int kTileCols = kChunks * 32;        // 256
constexpr int kRowLanes = kThreads / kChunks;  // 32
constexpr int kRedStride = 36;                 // LDS floats per chunk (padded)
constexpr int kRedRow = kChunks * kRedStride;  // LDS floats per row-lane
// MoE decode gate_up tiles are 256 columns wide (gate 128 | up 128 of the
// same 128 act columns, two 64-byte pieces of every weight row); 32 row-lanes
// of 8 rows: 256-row K-slices, so a reduction over the slices is one batch of
// device-coherent loads per column.
constexpr int kGuChunks = 8;
constexpr int kGuTileCols = kGuChunks * 32;      // 256
constexpr int kGuActCols = kGuTileCols / 2;      // 128
constexpr int kGuRowLanes = kThreads / kGuChunks;
constexpr int kGuL = 8;
// MoE decode down tiles: every act row in one workgroup, in passes of
// (kThreads / CH) row-lanes x L rows, summed in pass order. The shape follows
// the token count (registers hold MR x 32 accumulators), in the fused and
// the separate launch alike: one token, 256 columns of 4 rows (128-row
// passes, the passes of the one-token XCD-group launch); two tokens, 256
// columns of 8 rows; three or four, 256 columns of 4.
// With 64-column tiles and H a multiple of 256, tile i covers columns
// 256*(i % G) + 64*(i / G), G = H/256: the four tiles of one 256-column
// group (one 128-byte line of every weight row) are G apart in index, so
// with G a multiple of 8 they run on one XCD and share its L2.
template <int MR>
constexpr int dn_rows_per_lane() { return MR == 1 ? 4 : (MR == 2 ? 8 : 4); }
template <int MR>
constexpr int dn_chunks() { return 8; }
template <int MR>
constexpr int dn_tile_cols() { return dn_chunks<MR>() * 32; }
QMOE_DEV int dn_col0(int tile, int tc, int H) {
  if (tc == 64 && (H & 255) == 0) {
    const int G = H >> 8;
    return (tile % G) * 256 + (tile / G) * 64;
  }
  return tile * tc;
}
constexpr int dn_mr_of(int B) { return B == 1 ? 1 : (B == 2 ? 2 : 4); }

// Byte-permute selectors for v_perm_b32(hi, lo, sel): bytes of the result,
// low to high, taken from {lo.b0..b3 = 0..3, hi.b0..b3 = 4..7}.
constexpr uint32_t kSelLo = 0x05040100u;  // lo.b0, lo.b1, hi.b0, hi.b1
constexpr uint32_t kSelHi = 0x07060302u;  // lo.b2, lo.b3, hi.b2, hi.b3

QMOE_DEV bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// Nibble j (0..3) of each 16-bit half of t (two's complement q) -> bf16 pair
// 16 + u = q + 24 with u = q + 8. The nibble is shifted to bits 3..6 of its
// half (the top mantissa bits); one v_bitop3 then flips its top bit (two's
// complement -> offset binary, now bit 6), keeps bits 3..6 and fills the
// rest of the half with the sign and exponent of bf16 16.0:
// f(s, a, b) = a ? b : s ^ b, with a = ~keep and b = (16.0 bits outside
// keep) | (the flipped bit inside it). The truth table byte is f evaluated
// on the operand patterns 0xF0, 0xCC, 0xAA.
constexpr uint32_t kNibKeepNot = ~0x00780078u;                // a: bits outside 3..6 of each half
constexpr uint32_t kNibFill = 0x41804180u | 0x00400040u;      // b: bf16 16.0 | flipped top bit
constexpr uint8_t kNibTable = (uint8_t)((0xCC & 0xAA) | (~0xCC & (0xF0 ^ 0xAA)));  // 0x9A
template <int J>
QMOE_DEV uint32_t nib_pair(uint32_t t) {
  const uint32_t s = (J == 0) ? (t << 3) : (t >> (4 * J - 3));
  return __builtin_amdgcn_bitop3_b32(s, kNibKeepNot, kNibFill, kNibTable);
}

// One row pair (words a from row k, b from row k+1) of a 32-column chunk:
// acc[m][c] += x[m][k] * W'[k,c] + x[m][k+1] * W'[k+1,c] (W' = q + 24).
template <int MR>
QMOE_DEV void dot_row_pair(const uint4& a, const uint4& b, const uint32_t* xp, float (*acc)[32]) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
  const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t tl = __builtin_amdgcn_perm(bw[w], aw[w], kSelLo);
    const uint32_t th = __builtin_amdgcn_perm(bw[w], aw[w], kSelHi);
    const uint32_t p[8] = {nib_pair<0>(tl), nib_pair<1>(tl), nib_pair<2>(tl), nib_pair<3>(tl),
                           nib_pair<0>(th), nib_pair<1>(th), nib_pair<2>(th), nib_pair<3>(th)};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
        acc[m][8 * w + j] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(p[j]), as_bf16x2(xp[m]),
                                                            acc[m][8 * w + j], false);
    }
  }
}

// Partial product of one workgroup: for m < MR and the tile's 256 columns,
//   out[m][col] = sum_{k in [k0, kend)} x[m][k] * q[k][col] * S[k/gs][col]
// written to red_out (LDS, [MR][256]) in column-tile order.
//  w     : int32 words of the [K, N/8] matrix (one expert)
//  s     : bf16 scales [G, N]
//  xr    : bf16 activation rows (row m at xr.p[m]); rows m >= mrows read as zero
//  colw  : first word (column/8) of this thread's chunk, or -1 if unused
struct XRows {
  const uint16_t* p[4];
};

// Weight words and scales of one thread's run, loaded ahead of the
// activations (the fused decode kernel issues them before it waits for its
// inputs).
template <int L>
struct TileLoad {
  uint4 wv[L];
  uint32_t sw[16];
  bool active;
  int kr;
};

// CH = 32-column chunks per row of the tile (2: 64 columns, 4: 128, 8: 256,
// 16: 512), so a thread is (row-lane tid / CH, chunk tid % CH) and
// kThreads / CH row-lanes split the K-slice.
template <int L, int CH = kChunks>
QMOE_DEV void tile_load(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s, int N, int gs, int k0,
                        int kend, int colw, TileLoad<L>& t) {
  const int tid = threadIdx.x;
  const int r = tid / CH;
  const int nw = N >> 3;
  t.kr = k0 + r * L;  // first row of this thread's run
  t.active = colw >= 0 && t.kr < kend;
  if (t.active) {
    const uint32_t* wp = w + (size_t)t.kr * nw + colw;
#pragma unroll
    for (int i = 0; i < L; ++i) t.wv[i] = *reinterpret_cast<const uint4*>(wp + (size_t)i * nw);
    // scale group of this run (a run lies in one group)
    const uint4* sp = reinterpret_cast<const uint4*>(s + (size_t)(t.kr / gs) * N + (size_t)colw * 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = sp[q];
      t.sw[4 * q] = v.x; t.sw[4 * q + 1] = v.y; t.sw[4 * q + 2] = v.z; t.sw[4 * q + 3] = v.w;
    }
  }
}

// Activations of one thread's run: bf16 pairs (x[m][kr+2i], x[m][kr+2i+1])
// and their sum. AGENT_X reads x with device-coherent loads (x written by
// other workgroups of the launch). Rows m >= mrows and inactive runs read as
// zero.
template <int MR, int L>
struct XLoad {
  uint32_t xp[MR][L / 2];
};

template <int MR, int L, bool AGENT_X>
QMOE_DEV void x_load(const XRows& xr, int mrows, int kr, bool active, XLoad<MR, L>& xl) {
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int i = 0; i < L / 2; ++i) {
      uint32_t v = 0u;
      if (active && m < mrows) {
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(xr.p[m] + kr + 2 * i);
        v = AGENT_X ? __hip_atomic_load(const_cast<uint32_t*>(xa), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *xa;
      }
      xl.xp[m][i] = v;
    }
  }
}

// Partial product of one workgroup from loaded weights: for m < MR and the
// tile's CH*32 columns,
//   out[m][col] = sum_{k in [k0, kend)} x[m][k] * q[k][col] * S[k/gs][col]
// written to red_out (LDS, [MR][CH*32]) in column-tile order.
template <int MR, int L, int CH = kChunks>
QMOE_DEV void tile_compute_x(const TileLoad<L>& t, const XLoad<MR, L>& xl, float* red, float* red_out) {
  static_assert(CH == 2 || CH == 4 || CH == 8 || CH == 16, "64- to 512-column tiles");
  constexpr int kLanes = kThreads / CH;     // row-lanes
  constexpr int kRow = CH * kRedStride;     // LDS floats per row-lane
  static_assert(kLanes * kRow == kRowLanes * kRedRow, "same LDS footprint for both tile widths");
  const int tid = threadIdx.x;
  const int cc = tid & (CH - 1);
  const int r = tid / CH;

  float acc[MR][32];
  if (t.active) {
    float sx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      sx[m] = 0.f;
#pragma unroll
      for (int i = 0; i < L / 2; ++i) sx[m] += bf16_to_f32(xl.xp[m][i] & 0xffffu) + bf16_to_f32(xl.xp[m][i] >> 16);
#pragma unroll
      for (int c = 0; c < 32; ++c) acc[m][c] = -24.f * sx[m];
    }
#pragma unroll
    for (int i = 0; i < L / 2; ++i) {
      uint32_t xpi[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) xpi[m] = xl.xp[m][i];
      dot_row_pair<MR>(t.wv[2 * i], t.wv[2 * i + 1], xpi, acc);
    }
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const float sc = bf16_to_f32((c & 1) ? (t.sw[c >> 1] >> 16) : (t.sw[c >> 1] & 0xffffu));
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m][c] *= sc;
    }
  } else {
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < 32; ++c) acc[m][c] = 0.f;
  }

  // deterministic reduction over the row-lanes, one row of x at a time
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float4* dst = reinterpret_cast<float4*>(red + r * kRow + cc * kRedStride);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      dst[q] = make_float4(acc[m][4 * q], acc[m][4 * q + 1], acc[m][4 * q + 2], acc[m][4 * q + 3]);
    __syncthreads();
    if constexpr (CH * 32 >= kThreads) {
#pragma unroll
      for (int h = 0; h < CH * 32 / kThreads; ++h) {
        const int col = tid + kThreads * h;
        const float* src = red + (col >> 5) * kRedStride + (col & 31);
        float sum = 0.f;
#pragma unroll 8
        for (int rr = 0; rr < kLanes; ++rr) sum += src[rr * kRow];
        red_out[m * CH * 32 + col] = sum;
      }
    } else {
      // narrow tiles: kG groups of row-lanes summed in parallel, then the
      // group sums in group order
      constexpr int kCols = CH * 32, kG = kThreads / kCols, kPer = kLanes / kG;
      __shared__ float s_grp[kThreads];
      const int col = tid % kCols, g = tid / kCols;
      const float* src = red + (col >> 5) * kRedStride + (col & 31) + g * kPer * kRow;
      float sum = 0.f;
#pragma unroll 8
      for (int rr = 0; rr < kPer; ++rr) sum += src[rr * kRow];
      s_grp[tid] = sum;
      __syncthreads();
      if (tid < kCols) {
        float tot = 0.f;
#pragma unroll
        for (int q = 0; q < kG; ++q) tot += s_grp[q * kCols + tid];
        red_out[m * kCols + tid] = tot;
      }
    }
    __syncthreads();
  }
}

template <int MR, int L, bool AGENT_X, int CH = kChunks>
QMOE_DEV void tile_compute(const TileLoad<L>& t, const XRows& xr, int mrows, float* red, float* red_out) {
  XLoad<MR, L> xl;
  x_load<MR, L, AGENT_X>(xr, mrows, t.kr, t.active, xl);
  tile_compute_x<MR, L, CH>(t, xl, red, red_out);
}

template <int MR, int L>
QMOE_DEV void w4_tile_partial(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                              const XRows& xr, int mrows, int K, int N,
                              int gs, int k0, int kend, int colw, float* red, float* red_out) {
  (void)K;
  TileLoad<L> t;
  tile_load<L>(w, s, N, gs, k0, kend, colw, t);
  tile_compute<MR, L, false>(t, xr, mrows, red, red_out);
}

// Down projection of one CH*32-column tile over all MI act rows: passes of
// (kThreads/CH)*L rows (the first one's weights already in tl), each reduced
// over the row-lanes, summed in pass order into y[m] (column threadIdx.x,
// meaningful below CH*32). MR rows of act are computed (mrows of them real).
template <int MR, int L, int CH>
QMOE_DEV void down_tile(const uint32_t* __restrict__ we, const uint16_t* __restrict__ se, int H, int MI, int gs,
                        int colw, TileLoad<L>& tl, const XRows& xr, int mrows, float* red, float* res, float* y) {
  constexpr int kRows = (kThreads / CH) * L, kCols = CH * 32;
  const int c = min((int)threadIdx.x, kCols - 1);
  for (int p = 0;; ++p) {
    tile_compute<MR, L, false, CH>(tl, xr, mrows, red, res);
#pragma unroll
    for (int m = 0; m < MR; ++m) y[m] = (p == 0) ? res[m * kCols + c] : y[m] + res[m * kCols + c];
    if ((p + 1) * kRows >= MI) break;
    tile_load<L, CH>(we, se, H, gs, (p + 1) * kRows, min(MI, (p + 2) * kRows), colw, tl);
  }
}

// Narrow tiles: 256 columns as 32 chunks of 8 (one int32 word per row) x 8
// row-lanes of R rows (8R rows per workgroup); thread = (row-lane tid / 32,
// chunk tid % 32). Few accumulators per thread keep the cross-lane
// reduction small next to the dot products.
constexpr int kNarrowChunks = 32;
constexpr int kNarrowLanes = kThreads / kNarrowChunks;  // 8
constexpr int kNarrowR = 16;                             // rows per thread
constexpr int kNarrowRows = kNarrowLanes * kNarrowR;     // 128 rows per narrow slice or pass
// gate_up K-slices of the one-token decode (both launch forms) are 128 rows
// (256-row ones measured slower): 16 rows per thread, or where the group
// size is not a multiple of 16, two 64-row halves of 8 rows per thread
// summed in order (a thread's rows lie in one scale group).
QMOE_HOST_DEV constexpr int gu_rows_per_lane(int gs) { return (gs % 16) == 0 ? 16 : 8; }

template <int N>
struct IntConst {
  static constexpr int value = N;
};

// Word column of narrow gate_up chunk cc (gate 128 | up 128 of act tile m).
QMOE_DEV int narrow_gu_colw(int cc, int m, int MI) {
  return (cc < kNarrowChunks / 2) ? 16 * m + cc : (MI >> 3) + 16 * m + (cc - kNarrowChunks / 2);
}

template <int R>
struct NarrowLoad {
  uint32_t w[R];
  uint4 sc;  // the 8 columns' bf16 scales of the run's group
};

// Rows [k0 + R r, k0 + R r + R) of word column colw (all inside one scale group).
template <int R>
QMOE_DEV void narrow_load(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s, int N, int gs, int k0,
                          int colw, NarrowLoad<R>& t) {
  const int kr = k0 + (int)(threadIdx.x / kNarrowChunks) * R;
  const uint32_t* wp = w + (size_t)kr * (N >> 3) + colw;
#pragma unroll
  for (int i = 0; i < R; ++i) t.w[i] = __builtin_nontemporal_load(wp + (size_t)i * (N >> 3));  // read once
  t.sc = load_nt16(s + (size_t)(kr / gs) * N + (size_t)colw * 8);
}

// The same words from a decode tile: tb is the thread's first word of the
// run in the workgroup's 16 KB block (row word p of thread t at p * 256 + t).
constexpr int kDecodeTileWords = kThreads * kNarrowR;  // 4096
template <int R>
QMOE_DEV void narrow_load_tiled(const uint32_t* __restrict__ tb, const uint16_t* __restrict__ s, int N, int gs,
                                int k0, int colw, NarrowLoad<R>& t) {
  const int kr = k0 + (int)(threadIdx.x / kNarrowChunks) * R;
#pragma unroll
  for (int i = 0; i < R; ++i) t.w[i] = __builtin_nontemporal_load(tb + i * kThreads + threadIdx.x);  // read once
  t.sc = load_nt16(s + (size_t)(kr / gs) * N + (size_t)colw * 8);
}

// tile_load from decode tiles (the one-token launch's layout, see
// decode_tiles_kernel): te is the expert's tiles, per128 the tiles per
// 128-row slice (gate_up: act tiles t1; down: column tiles t2), tc this
// workgroup's tile in the slice, gr the rows per lane the tiles were built
// with, w0 the thread's first word in the tile row (16-byte aligned). Row R
// of the run is word p * 256 + r8 * 32 + w0 of tile (R / 128) * per128 + tc
// (p, r8 from R % 128 and gr). The 8 row-lanes of a wave read 1 KB in one
// piece per row. Scales as tile_load.
template <int L, int CH = kChunks>
QMOE_DEV void tile_load_dtile(const uint32_t* __restrict__ te, int per128, int tc, int gr, int w0,
                              const uint16_t* __restrict__ s, int N, int gs, int k0, int kend, int colw,
                              TileLoad<L>& t) {
  const int tid = threadIdx.x;
  const int r = tid / CH;
  t.kr = k0 + r * L;
  t.active = colw >= 0 && t.kr < kend;
  if (t.active) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const int R = t.kr + i, q = R & (kNarrowRows - 1);
      const int h = q / (kNarrowLanes * gr), r8 = (q % (kNarrowLanes * gr)) / gr, pp = h * gr + q % gr;
      t.wv[i] = *reinterpret_cast<const uint4*>(te + (size_t)((R / kNarrowRows) * per128 + tc) * kDecodeTileWords +
                                                pp * kThreads + r8 * kNarrowChunks + w0);
    }
    const uint4* sp = reinterpret_cast<const uint4*>(s + (size_t)(t.kr / gs) * N + (size_t)colw * 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = sp[q];
      t.sw[4 * q] = v.x; t.sw[4 * q + 1] = v.y; t.sw[4 * q + 2] = v.z; t.sw[4 * q + 3] = v.w;
    }
  }
}

// The thread's weights as bf16 pairs (W'[k, col], W'[k + 1, col]) with
// W' = q + 24, rows in pairs, 8 columns: independent of the activations, so
// a workgroup that waits for them unpacks first.
template <int R>
struct NarrowPairs {
  uint32_t p[R / 2][8];
  uint4 sc;
};

template <int R>
QMOE_DEV void narrow_unpack(const NarrowLoad<R>& t, NarrowPairs<R>& u) {
#pragma unroll
  for (int i = 0; i < R / 2; ++i) {
    const uint32_t tl = __builtin_amdgcn_perm(t.w[2 * i + 1], t.w[2 * i], kSelLo);
    const uint32_t th = __builtin_amdgcn_perm(t.w[2 * i + 1], t.w[2 * i], kSelHi);
    u.p[i][0] = nib_pair<0>(tl); u.p[i][1] = nib_pair<1>(tl); u.p[i][2] = nib_pair<2>(tl); u.p[i][3] = nib_pair<3>(tl);
    u.p[i][4] = nib_pair<0>(th); u.p[i][5] = nib_pair<1>(th); u.p[i][6] = nib_pair<2>(th); u.p[i][7] = nib_pair<3>(th);
  }
  u.sc = t.sc;
}

// out = sum over the 8R rows of x[k] * q[k][col] * S[k/gs][col] for the
// tile's 256 columns, column threadIdx.x (row-lane partials summed in
// row-lane order through LDS). xp: the thread's R/2 bf16 pairs of x.
template <int R>
QMOE_DEV float narrow_dots(const NarrowPairs<R>& u, const uint32_t* xp, float* red) {
  float sx = 0.f;
#pragma unroll
  for (int i = 0; i < R / 2; ++i) sx += bf16_to_f32(xp[i] & 0xffffu) + bf16_to_f32(xp[i] >> 16);
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = -24.f * sx;
#pragma unroll
  for (int i = 0; i < R / 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc[j] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(u.p[i][j]), as_bf16x2(xp[i]), acc[j], false);
  const uint32_t sw[4] = {u.sc.x, u.sc.y, u.sc.z, u.sc.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] *= bf16_to_f32((j & 1) ? (sw[j >> 1] >> 16) : (sw[j >> 1] & 0xffffu));
  float4* dst = reinterpret_cast<float4*>(red + threadIdx.x * 8);  // (row-lane, chunk, column) = 256 r + 8 cc + j
  dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  __syncthreads();
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < kNarrowLanes; ++r) sum += red[r * 256 + threadIdx.x];
  __syncthreads();
  return sum;
}

template <int R>
QMOE_DEV float narrow_compute(const NarrowLoad<R>& t, const uint32_t* xp, float* red) {
  NarrowPairs<R> u;
  narrow_unpack<R>(t, u);
  return narrow_dots<R>(u, xp, red);
}

// ---------------------------------------------------------------- fused MoE decode

constexpr int kMaxTok = 4;                     // tokens per decode call
constexpr int kMaxSlots = kMaxTok * QMOE_KMAX;  // routed (token, slot) pairs

// Routing plan shared by the two decode kernels (lives in the workspace).
struct DecodePlan {
  int nunique;                    // distinct experts among the routed pairs
  int uexp[kMaxSlots];            // expert id of unique slot u
  int umult[kMaxSlots];           // tokens routed to it (<= kMaxTok)
  int utok[kMaxSlots][kMaxTok];   // those tokens, ascending
  int uslot[kMaxSlots][kMaxTok];  // the top-k slot each of them used
  float w[kMaxTok][QMOE_KMAX];    // bf16-rounded routing weights (as fp32)
  int urow[kMaxSlots];            // first (u, m) row of unique slot u: sum of umult[v < u]
};

// Plan of one token from a selection every wave holds (sel, one rank per
// lane) and the logits lg of wave_route_keys, which wave rwave holds: that
// wave computes the softmax weights; unique slot u = top-k slot u. Contains
// barriers (call from the whole workgroup). KPL: logits per lane of lg.
template <int KPL = 8>
QMOE_DEV void plan_one_token(const float* lg, int E, int k, uint32_t sel, int rwave, DecodePlan& plan,
                             int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out, bool write_out) {
  __shared__ int s_idx1[QMOE_KMAX];
  __shared__ float s_w1[QMOE_KMAX];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  if (wave == rwave) wave_route_softmax<KPL>(lg, E, k, sel, s_idx1, s_w1);
  __syncthreads();
  if (wave == 0) {
    if (lane < k) {
      const int e = s_idx1[lane];
      plan.uexp[lane] = e;
      plan.umult[lane] = 1;
      plan.utok[lane][0] = 0;
      plan.uslot[lane][0] = lane;
      plan.urow[lane] = lane;
      const uint32_t wb = f32_to_bf16(s_w1[lane]);
      plan.w[0][lane] = bf16_to_f32(wb);
      if (write_out) {
        idx_out[lane] = e;
        w_out[lane] = (uint16_t)wb;
      }
    }
    if (lane == 0) plan.nunique = k;
  }
  __syncthreads();
}

// Router for B tokens (one wave each, waves 0..3) plus expert
// de-duplication. Every workgroup computes the same plan into LDS. The
// de-duplication runs in wave 0 with ballots: each round takes the first
// unplaced (token, slot) pair, gathers every pair with the same expert (in
// pair order) and gives them the next unique index.
template <int KPL>
QMOE_DEV void build_plan(const uint16_t* __restrict__ logits, int B, int E, int k, DecodePlan& plan,
                         int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out, bool write_out) {
  __shared__ int s_idx[kMaxTok * QMOE_KMAX];
  __shared__ float s_w[kMaxTok * QMOE_KMAX];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  if (wave < B)
    wave_topk_softmax<KPL>(logits + (size_t)wave * E, E, k, s_idx + wave * QMOE_KMAX, s_w + wave * QMOE_KMAX);
  __syncthreads();
  if (wave == 0 && B == 1) {
    // one token: its k experts are distinct, unique slot u = top-k slot u
    if (lane < k) {
      const int e = s_idx[lane];
      plan.uexp[lane] = e;
      plan.umult[lane] = 1;
      plan.utok[lane][0] = 0;
      plan.uslot[lane][0] = lane;
      plan.urow[lane] = lane;
      const uint32_t wb = f32_to_bf16(s_w[lane]);
      plan.w[0][lane] = bf16_to_f32(wb);
      if (write_out) {
        idx_out[lane] = e;
        w_out[lane] = (uint16_t)wb;
      }
    }
    if (lane == 0) plan.nunique = k;
  } else if (wave == 0) {
    const int n = B * k;  // <= 64
    const bool valid = lane < n;
    const int t = valid ? lane / k : 0, j = valid ? lane % k : 0;
    const int e = valid ? s_idx[t * QMOE_KMAX + j] : -1;
    uint64_t remaining = __builtin_amdgcn_ballot_w64(valid);
    int u = 0, row = 0;
    while (remaining != 0) {
      const int leader = __builtin_ctzll(remaining);
      const int el = __builtin_amdgcn_readlane(e, leader);
      const uint64_t match = __builtin_amdgcn_ballot_w64(valid && e == el);
      if ((match >> lane) & 1ull) {
        const int m = __builtin_popcountll(match & ((1ull << lane) - 1ull));
        if (m == 0) {
          plan.uexp[u] = e;
          plan.umult[u] = __builtin_popcountll(match);
          plan.urow[u] = row;
        }
        plan.utok[u][m] = t;
        plan.uslot[u][m] = j;
      }
      remaining &= ~match;
      row += __builtin_popcountll(match);
      ++u;
    }
    if (valid) {
      const uint32_t wb = f32_to_bf16(s_w[t * QMOE_KMAX + j]);
      plan.w[t][j] = bf16_to_f32(wb);
      if (write_out) {
        idx_out[(size_t)t * k + j] = e;
        w_out[(size_t)t * k + j] = (uint16_t)wb;
      }
    }
    if (lane == 0) plan.nunique = u;
  }
  __syncthreads();
}

// Phase 1: gate_up projection of every (unique expert, token) row, then
// SwiGLU: act = bf16(silu(bf16(g)) * bf16(u)) with g = column i, u = MI + i.
// grid.x = (MI/128 act-column tiles) x (256-row K-slices), grid.y = B*k
// unique slots; the same tiles and summation order as the fused launch.
template <int L>
__global__ __launch_bounds__(kThreads) void moe_decode_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ logits, const uint32_t* __restrict__ wgu,
    const uint16_t* __restrict__ sgu, int B, int E, int k, int H, int MI, int gs,
    DecodePlan* __restrict__ gplan, float* __restrict__ part, uint16_t* __restrict__ act,
    int* __restrict__ counters, int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out) {
  static_assert(L == kGuL, "fused and separate gate_up share their slices");
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[kMaxTok * kGuTileCols];
  __shared__ DecodePlan plan;
  const int ntiles = ceil_div(MI, kGuActCols);
  const int tile = blockIdx.x % ntiles;
  const int slice = blockIdx.x / ntiles;
  const int nslices = gridDim.x / ntiles;
  const int u = blockIdx.y;
  const bool writer = (blockIdx.x == 0 && u == 0);
  if (E <= 512) build_plan<8>(logits, B, E, k, plan, idx_out, w_out, writer);
  else build_plan<16>(logits, B, E, k, plan, idx_out, w_out, writer);
  if (writer) {
    // publish the plan for phase 2 (plain stores; the kernel boundary orders them)
    const int* src = reinterpret_cast<const int*>(&plan);
    int* dst = reinterpret_cast<int*>(gplan);
    for (int q = threadIdx.x; q < (int)(sizeof(DecodePlan) / sizeof(int)); q += kThreads) dst[q] = src[q];
  }
  if (u >= plan.nunique) return;
  const int e = plan.uexp[u];
  const int mult = plan.umult[u];
  const int N = 2 * MI;
  if (B == 1 && (H % kTileCols) == 0 && (MI % kGuActCols) == 0) {
    // the slices of the one-token XCD-group launch: 128-row narrow tiles,
    // summed in slice order by the last to arrive
    const uint32_t* we = wgu + (size_t)e * H * (N >> 3);
    const uint16_t* se = sgu + (size_t)e * (H / gs) * N;
    auto slice_sum = [&](auto r_c) -> float {
      constexpr int R = decltype(r_c)::value;
      float v = 0.f;
      for (int h = 0; h < kNarrowRows / (kNarrowLanes * R); ++h) {
        const int k0 = slice * kNarrowRows + h * kNarrowLanes * R;
        NarrowLoad<R> nl;
        narrow_load<R>(we, se, N, gs, k0, narrow_gu_colw(threadIdx.x % kNarrowChunks, tile, MI), nl);
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(x + k0 + (threadIdx.x / kNarrowChunks) * R);
        uint32_t xp[R / 2];
#pragma unroll
        for (int i = 0; i < R / 2; ++i) xp[i] = xa[i];
        v += narrow_compute<R>(nl, xp, red);
      }
      return v;
    };
    const float v = gu_rows_per_lane(gs) == 16 ? slice_sum(IntConst<16>{}) : slice_sum(IntConst<8>{});
    const size_t tile_stride = (size_t)ntiles * kGuTileCols;
    float* mypart = part + (((size_t)u * nslices + slice) * kMaxTok) * tile_stride + (size_t)tile * kGuTileCols;
    store_agent(&mypart[threadIdx.x], v);
    if (!arrive_last(counters + u * ntiles + tile, nslices)) return;
    const int i = threadIdx.x;
    if (i >= kGuActCols) return;
    const float* p = part + ((size_t)u * nslices * kMaxTok) * tile_stride + (size_t)tile * kGuTileCols;
    const float g = sum_agent_ordered(p + i, kMaxTok * tile_stride, nslices);
    const float up = sum_agent_ordered(p + kGuActCols + i, kMaxTok * tile_stride, nslices);
    act[(size_t)u * kMaxTok * MI + tile * kGuActCols + i] =
        (uint16_t)f32_to_bf16(silu_f32(round_bf16(g)) * round_bf16(up));
    return;
  }
  const int cc = threadIdx.x & (kGuChunks - 1);
  const int ic = tile * kGuActCols + (cc & (kGuChunks / 2 - 1)) * 32;  // intermediate column of the chunk
  const int col0 = (cc < kGuChunks / 2) ? ic : MI + ic;
  const int colw = ic < MI ? (col0 >> 3) : -1;

  // rows of x of the tokens routed to this expert
  XRows xr;
#pragma unroll
  for (int m = 0; m < kMaxTok; ++m) xr.p[m] = x + (size_t)plan.utok[u][min(m, mult - 1)] * H;

  const uint32_t* we = wgu + (size_t)e * H * (N >> 3);
  const uint16_t* se = sgu + (size_t)e * (H / gs) * N;
  const int ks = kGuRowLanes * L;
  const int k0 = slice * ks;
  const int kend = min(H, k0 + ks);
  TileLoad<L> tl;
  tile_load<L, kGuChunks>(we, se, N, gs, k0, kend, colw, tl);
  if (mult == 1) tile_compute<1, L, false, kGuChunks>(tl, xr, 1, red, res);
  else if (mult == 2) tile_compute<2, L, false, kGuChunks>(tl, xr, 2, red, res);
  else tile_compute<4, L, false, kGuChunks>(tl, xr, mult, red, res);

  // partials: part[u][slice][m][tile][512]
  const size_t tile_stride = (size_t)ntiles * kGuTileCols;
  float* mypart = part + (((size_t)u * nslices + slice) * kMaxTok) * tile_stride + (size_t)tile * kGuTileCols;
  for (int m = 0; m < mult; ++m)
#pragma unroll
    for (int h = 0; h < kGuTileCols / kThreads; ++h)
      store_agent(&mypart[(size_t)m * tile_stride + h * kThreads + threadIdx.x], res[m * kGuTileCols + h * kThreads + threadIdx.x]);
  if (!arrive_last(counters + u * ntiles + tile, nslices)) return;

  // last workgroup of this (expert, tile): reduce slices, SwiGLU, store act
  const int i = threadIdx.x;
  const int col = tile * kGuActCols + i;
  if (i >= kGuActCols) return;
  for (int m = 0; m < mult; ++m) {
    const float* p = part + ((size_t)u * nslices * kMaxTok + m) * tile_stride + (size_t)tile * kGuTileCols;
    const float g = sum_agent_ordered(p + i, kMaxTok * tile_stride, nslices);
    const float up = sum_agent_ordered(p + kGuActCols + i, kMaxTok * tile_stride, nslices);
    if (col < MI) {
      const float gb = round_bf16(g), ub = round_bf16(up);
      act[((size_t)u * kMaxTok + m) * MI + col] = (uint16_t)f32_to_bf16(silu_f32(gb) * ub);
    }
  }
}

// Phase 2: down projection of every (unique expert, token) act row, then the
// fused top-k combine: prod = bf16(bf16(y) * w), out = bf16(sum_j prod_j in
// slot order) and, when a shared expert is given, the shared merge
// out = bf16(out + bf16(shared * bf16(sigmoid(gate)))).
// grid.x = H/256 column tiles, grid.y = B*k unique slots; each workgroup
// covers all MI act rows (the same passes as the fused launch: MRB = the
// accumulator rows the fused launch uses for this B).
template <int MRB>
__global__ __launch_bounds__(kThreads) void moe_decode_down_kernel(
    const uint32_t* __restrict__ wdn, const uint16_t* __restrict__ sdn, int B, int k, int H, int MI,
    int gs, const DecodePlan* __restrict__ gplan, const uint16_t* __restrict__ act,
    float* __restrict__ prod, int* __restrict__ counters_out, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ out) {
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[kMaxTok * kTileCols];
  __shared__ DecodePlan plan;
  {
    const int* src = reinterpret_cast<const int*>(gplan);
    int* dst = reinterpret_cast<int*>(&plan);
    for (int q = threadIdx.x; q < (int)(sizeof(DecodePlan) / sizeof(int)); q += kThreads) dst[q] = src[q];
    __syncthreads();
  }
  constexpr int CH = dn_chunks<MRB>(), TC = dn_tile_cols<MRB>();
  const int tile = blockIdx.x;
  const int u = blockIdx.y;
  const int nunique = plan.nunique;
  if (u >= nunique) return;
  const int e = plan.uexp[u];
  const int mult = plan.umult[u];
  const int cc = threadIdx.x & (CH - 1);
  const int tcol = dn_col0(tile, TC, H);
  const int col0 = tcol + cc * 32;
  const int colw = col0 < H ? (col0 >> 3) : -1;
  const uint32_t* we = wdn + (size_t)e * MI * (H >> 3);
  const uint16_t* se = sdn + (size_t)e * (MI / gs) * H;
  XRows xr;
#pragma unroll
  for (int m = 0; m < kMaxTok; ++m) xr.p[m] = act + ((size_t)u * kMaxTok + min(m, mult - 1)) * MI;
  if constexpr (MRB == 1) {
    if ((H % kTileCols) == 0 && (MI % 128) == 0) {
      // the passes of the one-token XCD-group launch: 128-row narrow tiles
      // summed in pass order
      const uint16_t* a = act + (size_t)u * kMaxTok * MI;
      const int cw = tile * (kTileCols / 8) + (int)(threadIdx.x % kNarrowChunks);
      float yy = 0.f;
      for (int p = 0; p * 128 < MI; ++p) {
        NarrowLoad<16> nl;
        narrow_load<16>(we, se, H, gs, p * 128, cw, nl);
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(a + p * 128 + (threadIdx.x / kNarrowChunks) * 16);
        uint32_t xp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xp[i] = xa[i];
        const float yp = narrow_compute<16>(nl, xp, red);
        yy = (p == 0) ? yp : yy + yp;
      }
      const int t = plan.utok[u][0], j = plan.uslot[u][0];
      const int cl = tile * kTileCols + threadIdx.x;
      store_agent(&prod[((size_t)t * k + j) * H + cl], round_bf16(round_bf16(yy) * plan.w[t][j]));
      if (!arrive_last(counters_out + tile, nunique)) return;
      for (int tt = 0; tt < B; ++tt) {
        float acc = 0.f;
        for (int jj = 0; jj < k; ++jj) acc += load_agent(&prod[((size_t)tt * k + jj) * H + cl]);
        float r = round_bf16(acc);
        if (shared != nullptr) {
          const float g = bf16_to_f32(gate[tt]);
          const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
          r = round_bf16(r + round_bf16(bf16_to_f32(shared[(size_t)tt * H + cl]) * sg));
        }
        out[(size_t)tt * H + cl] = (uint16_t)f32_to_bf16(r);
      }
      return;
    }
  }
  constexpr int L = dn_rows_per_lane<MRB>();
  TileLoad<L> tl;
  tile_load<L, CH>(we, se, H, gs, 0, min(MI, (kThreads / CH) * L), colw, tl);
  float y[MRB];
  if (MRB == 1 || mult == 1) down_tile<1, L, CH>(we, se, H, MI, gs, colw, tl, xr, 1, red, res, y);
  else if (MRB == 2 || mult == 2) down_tile<(MRB >= 2 ? 2 : 1), L, CH>(we, se, H, MI, gs, colw, tl, xr, mult, red, res, y);
  else down_tile<MRB, L, CH>(we, se, H, MI, gs, colw, tl, xr, mult, red, res, y);

  // expert output of this tile -> weighted bf16 products at (token, slot)
  const int col = tcol + threadIdx.x;
  const bool mine = (int)threadIdx.x < TC && col < H;
  for (int m = 0; m < mult; ++m) {
    const int t = plan.utok[u][m], j = plan.uslot[u][m];
    if (mine) store_agent(&prod[((size_t)t * k + j) * H + col], round_bf16(round_bf16(y[m]) * plan.w[t][j]));
  }
  if (!arrive_last(counters_out + tile, nunique)) return;

  // every expert of every token has contributed this tile: ordered combine
  if (!mine) return;
  for (int t = 0; t < B; ++t) {
    // all k products in flight at once, then summed in slot order
    float pv[QMOE_KMAX];
#pragma unroll
    for (int j = 0; j < QMOE_KMAX; ++j) pv[j] = (j < k) ? load_agent(&prod[((size_t)t * k + j) * H + col]) : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < QMOE_KMAX; ++j)
      if (j < k) acc += pv[j];
    float r = round_bf16(acc);
    if (shared != nullptr) {
      const float g = bf16_to_f32(gate[t]);
      const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
      r = round_bf16(r + round_bf16(bf16_to_f32(shared[(size_t)t * H + col]) * sg));
    }
    out[(size_t)t * H + col] = (uint16_t)f32_to_bf16(r);
  }
}

// ---------------------------------------------------------------- fused single-launch decode
//
// One launch for the whole block. Blocks [0, n_gu) are gate_up workgroups
// (unique slot u, tile of 128 act columns read as gate 128 | up 128, 256-row
// K-slice of H). Blocks [n_gu, grid) are down workgroups (u, 256-column tile
// of H, all MI act rows). Cross-workgroup data travels through a mailbox as
// 64-bit words {payload, tag}, where tag = launch epoch + 1 marks a word as
// written by this launch: the data carries its own readiness, so no store
// has to be acknowledged and no counter bumped before a consumer can go on.
//  1. gate_up workgroups route (one wave selects the top-k of the token; on
//     the per-pair path with several tokens one workgroup per token then
//     publishes every pair's expert and routing weight as a tagged plan
//     word), load their weights
//     at once, and store their split-K partials
//     (fp32) as tagged words. The last of the K-slices of each (u, tile)
//     (arrival counter) then reads all of them (until every tag is this
//     launch's), sums them in slice order, applies SwiGLU and publishes the
//     128 act rows as tagged words of bf16 pairs.
//  2. Down workgroup (u, tile) loads its weights at once (per-pair path:
//     once the plan word of u is in; they depend only on
//     the routing), polls all act rows of u, computes its down tile over
//     every act row and stores the weighted products bf16(bf16(y) * w) as
//     tagged words.
//  3. The workgroup of the last unique slot of each tile combines: it polls
//     the k products of every token at its columns and sums them in slot
//     order (plus the shared merge). On the per-pair path (up to 512
//     experts, the one-row kernel for 1..4 tokens: units are (token, slot)
//     pairs) the last slot of each token combines that token.
// Workgroups are dispatched in index order and every wait is on workgroups
// that have already arrived (the reducing gate_up workgroup) or have lower
// indices, so the launch completes whatever the residency; every wait is also
// bounded and leaves an error flag instead of hanging.
//
// Epoch: a word of the counters array itself (slot kMailboxBase - 2), read
// by every workgroup when it starts. The last of the combiners (t2, or B*t2
// on the per-pair path; counted on cnt_rdy) advances it; by then every down
// workgroup has published its products and every gate_up one has been
// waited for, so all workgroups of the launch read the same value. Tags only
// grow (by one per launch), so words left by earlier launches, of any shape,
// never carry the current tag; the mailbox starts zeroed (tag 0). Each
// counters array has its own epoch, mailbox and flag: launches that overlap
// on two streams are independent when they use different arrays.
//
// Counters (int32): cnt_rdy at 0 and cnt_gu[B*k][t1] from kFlagStride on
// (128 bytes apart), returned to zero; the epoch at kMailboxBase - 2; the
// error flag at kMailboxBase - 1; the mailbox from int kMailboxBase on:
// uint64 gate_up words [B*k rows][s1][t1][256], act words [B*k rows][t1][64],
// product words [B][k][H], plan words [B*k] (per-pair path); rows in
// (unique slot, token) order.
//
// Inspection copies (the routing plan, act rows and weighted products in the
// caller's workspace) are written only when a workspace is passed.
constexpr int kSpinLimit = 1 << 22;  // polls (one agent-scope load each, about a microsecond)
constexpr int kFlagStride = 32;      // ints between arrival counters (128 bytes)
constexpr int kMailboxBase = QMOE_DECODE_MAILBOX_BASE;  // int offset of the mailbox in the counters array
constexpr int kEpochSlot = kMailboxBase - 2;            // launch epoch of this counters array
constexpr int kErrSlot = kMailboxBase - 1;              // sticky timeout flag

QMOE_DEV uint64_t mail_word(float v, uint32_t tag) {
  return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}
QMOE_DEV float mail_value(uint64_t w) { return __uint_as_float((uint32_t)w); }
QMOE_DEV bool mail_ready(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

// sum_{i < n} value(p[i * stride]) in index order, each word once it carries
// `tag`. The words are read sixteen at a time; one not yet written is read
// again, at most `spins` times (then *err is set and the word is added as it
// is).
QMOE_DEV float sum_mail_ordered(const uint64_t* p, size_t stride, int n, uint32_t tag, int spins, int* err) {
  float s = 0.f;
  for (int b = 0; b < n; b += 16) {
    uint64_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = load_agent64(p + (size_t)min(b + i, n - 1) * stride);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (b + i < n) {
        int polls = 0;
        while (!mail_ready(v[i], tag)) {
          if (polls++ >= spins) {
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(2);
          v[i] = load_agent64(p + (size_t)(b + i) * stride);
        }
        s += mail_value(v[i]);
      }
    }
  }
  return s;
}

// Block-wide wait until the words this thread names (n_mine of them at
// p[i * stride]) carry `tag`; their payloads go to out[i]. Polls are spaced
// and bounded (a timeout sets *err). Whole workgroup.
template <int NMAX>
QMOE_DEV void wait_mail_block(const uint64_t* p, size_t stride, int n_mine, uint32_t tag, uint32_t* out, int* err) {
  bool have[NMAX];
#pragma unroll
  for (int i = 0; i < NMAX; ++i) have[i] = i >= n_mine;
  int polls = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      if (!have[i]) {
        const uint64_t v = load_agent64(p + (size_t)i * stride);
        if (mail_ready(v, tag)) {
          out[i] = (uint32_t)v;
          have[i] = true;
        } else {
          ok = false;
        }
      }
    }
    if (__syncthreads_and(ok)) break;
    if (++polls == kSpinLimit) {
      if (threadIdx.x == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Largest MI the fused decode keeps in LDS as act rows.
constexpr int kMaxMI = 2048;

// Three workgroups per CU (LDS allows three; registers are held to 168 per
// lane) keep every workgroup of the one-token grid resident at once; the
// two- and four-token variants need more LDS and keep two.
template <int MRMAX, int L1 = kGuL, int DCH = dn_chunks<MRMAX>(), int DL = dn_rows_per_lane<MRMAX>()>
__global__ __launch_bounds__(kThreads, MRMAX == 1 ? 3 : 2) void moe_decode_fused_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ logits, const uint32_t* __restrict__ wgu,
    const uint16_t* __restrict__ sgu, const uint32_t* __restrict__ wdn, const uint16_t* __restrict__ sdn,
    const uint32_t* __restrict__ tgu, const uint32_t* __restrict__ tdn, int B,
    int E, int k, int H, int MI, int gs_gu, int gs_dn, int n_gu, DecodePlan* __restrict__ gplan,
    uint64_t* __restrict__ mbox, uint16_t* __restrict__ act, float* __restrict__ prod,
    int* __restrict__ counters, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ out, int64_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out) {
  uint32_t* epoch = reinterpret_cast<uint32_t*>(counters + kEpochSlot);
  int* err = counters + kErrSlot;
  const uint32_t tag = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  const bool inspect = gplan != nullptr;  // write the inspection copies
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[MRMAX * kGuTileCols];
  __shared__ DecodePlan plan;
  const int umax = B * k;
  constexpr int CH2 = DCH, TC2 = DCH * 32;
  const int t1 = ceil_div(MI, kGuActCols), s1 = ceil_div(H, kGuRowLanes * L1);
  const int t2 = ceil_div(H, TC2);
  int* cnt_rdy = counters;
  int* cnt_gu = counters + kFlagStride;  // one per (u, gate_up tile), 128 bytes apart

  const bool writer = blockIdx.x == 0;
  auto publish_plan = [&]() {
    const int* src = reinterpret_cast<const int*>(&plan);
    int* dst = reinterpret_cast<int*>(gplan);
    for (int q = threadIdx.x; q < (int)(sizeof(DecodePlan) / sizeof(int)); q += kThreads) dst[q] = src[q];
  };
  // fast path: the entries of token t (pairs t*k .. t*k + k-1) of the global
  // plan, from the one-token plan in LDS
  auto publish_plan_token = [&](int t) {
    const int j = threadIdx.x;
    if (j < k) {
      const int u = t * k + j;
      gplan->uexp[u] = plan.uexp[j];
      gplan->umult[u] = 1;
      gplan->utok[u][0] = t;
      gplan->uslot[u][0] = j;
      gplan->urow[u] = u;
      gplan->w[t][j] = plan.w[0][j];
    }
    if (t == 0 && j == 0) gplan->nunique = B * k;
  };
  // Fast path (E <= 512, this one-row kernel, 1..4 tokens): the units are
  // the (token, slot) pairs u = t*k + j themselves, not de-duplicated
  // experts. Every workgroup selects the top-k of its own token in one wave,
  // so it knows its expert without waiting for the softmax or a shared plan
  // and starts its weight loads at once; the weights and the inverse map are
  // built afterwards by the workgroups that need them, per token. An expert
  // picked by two tokens is streamed once per token.
  const bool fast = MRMAX == 1 && E <= 512;
  // gate_up geometry (from the block index alone): unique slot, act-column
  // tile and K-slice
  const bool is_gu = (int)blockIdx.x < n_gu;
  const int per_u = t1 * s1;
  // fast path: the token of this workgroup's pair (padding blocks past the
  // last pair take the last token and exit after routing)
  int tok = 0;
  if (fast && B > 1) {
    const int pair_of_block = is_gu ? (int)blockIdx.x / per_u : ((int)blockIdx.x - n_gu) / t2;
    tok = min(pair_of_block / k, B - 1);
  }
  int gu_u = 0, gu_tile = 0, gu_slice = 0;
  if (is_gu) {
    const int idx = blockIdx.x % per_u;
    gu_u = blockIdx.x / per_u;
    gu_tile = idx % t1;
    gu_slice = idx / t1;
    if ((t1 & 1) == 0 && (per_u & 15) == 0) {
      // tiles 2j and 2j+1 read the two halves of the same 128-byte lines:
      // give them indices 8 apart, so they run on one XCD and share its L2
      const int half = t1 >> 1, q = (idx & 7) + 8 * (idx >> 4);
      gu_slice = q / half;
      gu_tile = 2 * (q % half) + ((idx >> 3) & 1);
    }
  }
  const int gu_cc = threadIdx.x & (kGuChunks - 1);
  const int gu_ic = gu_tile * kGuActCols + (gu_cc & (kGuChunks / 2 - 1)) * 32;
  const int gu_colw = gu_ic < MI ? (((gu_cc < kGuChunks / 2) ? gu_ic : MI + gu_ic) >> 3) : -1;
  const int gu_k0 = gu_slice * (kGuRowLanes * L1), gu_kend = min(H, gu_k0 + kGuRowLanes * L1);
  // fast path: lane r holds the key of rank r; the routing wave (spread
  // over the SIMDs by block index) also holds the logits for the softmax.
  // With several tokens the down workgroups, which start late (after gate_up
  // ones have left the CUs) when the routing waves would contend with the
  // gate_up dot products, read their pair's plan word instead.
  const bool plan_words = fast && B > 1;
  uint32_t sel = 0u;
  float lgk[8];
  const int rwave = blockIdx.x & 3;
  if (fast && (is_gu || !plan_words)) {
    uint32_t key[8];
    // one wave per workgroup selects (the others would only contend for
    // its SIMD's issue slots); the selection goes to the others through LDS
    __shared__ uint32_t s_sel[QMOE_KMAX];
    if ((int)(threadIdx.x >> 6) == rwave) {
      wave_route_keys<8>(logits + (size_t)tok * E, E, key, lgk);
      sel = wave_route_select<8>(key, k);
      if ((threadIdx.x & 63) < QMOE_KMAX) s_sel[threadIdx.x & 63] = sel;
    }
    __syncthreads();
    sel = ((threadIdx.x & 63) < QMOE_KMAX) ? s_sel[threadIdx.x & 63] : 0u;
  } else if (!fast) {
    if (E <= 512) build_plan<8>(logits, B, E, k, plan, idx_out, w_out, writer);
    else build_plan<16>(logits, B, E, k, plan, idx_out, w_out, writer);
    if (writer && inspect) publish_plan();
  }
  auto sel_expert = [&](int u) { return route_key_expert(route_sel_rank(sel, u)); };
  const int nunique = fast ? B * k : plan.nunique;
  const size_t mrow = (size_t)s1 * t1 * kGuTileCols;  // gate_up words per (u, m) row
  const size_t act_words = (size_t)t1 * (kGuActCols / 2);  // act pair words per (u, m) row (whole tiles)
  uint64_t* abox_all = mbox + (size_t)umax * mrow;
  uint64_t* pbox = abox_all + (size_t)umax * act_words;  // product words [B][k][H]
  // fast path: per pair u, {expert | bf16 routing weight << 16} from the token's writer
  uint64_t* planbox = pbox + (size_t)B * k * H;

  if (is_gu) {
    // ---- gate_up partials
    const int u = gu_u, tile = gu_tile, slice = gu_slice;
    if (u >= nunique) return;
    const int e = fast ? sel_expert(u - tok * k) : plan.uexp[u];
    const int mult = fast ? 1 : plan.umult[u];
    const int urow = fast ? u : plan.urow[u];
    const int N = 2 * MI;
    const int colw = gu_colw;
    XRows xr;
#pragma unroll
    for (int m = 0; m < kMaxTok; ++m) xr.p[m] = x + (size_t)(fast ? tok : plan.utok[u][min(m, mult - 1)]) * H;
    const uint32_t* we = wgu + (size_t)e * H * (N >> 3);
    const uint16_t* se = sgu + (size_t)e * (H / gs_gu) * N;
    const int k0 = gu_k0, kend = gu_kend;
    TileLoad<L1> tl;
    if (fast && tgu != nullptr) {
      // decode tiles: chunk cc holds the gate words 4 cc .. 4 cc + 3 of the
      // tile row (cc < 4) or its up words 16 + 4 (cc - 4) ..
      const int cc = threadIdx.x & (kGuChunks - 1);
      const int w0 = (cc < kGuChunks / 2 ? 0 : 16) + 4 * (cc & (kGuChunks / 2 - 1));
      tile_load_dtile<L1, kGuChunks>(tgu + (size_t)e * H * (N >> 3), t1, tile, gu_rows_per_lane(gs_gu), w0, se, N,
                                     gs_gu, k0, kend, colw, tl);
    } else {
      tile_load<L1, kGuChunks>(we, se, N, gs_gu, k0, kend, colw, tl);
    }
    if (fast && u == tok * k && tile == 0 && slice == 0) {
      // the routing outputs of this token (one workgroup per token), while
      // this workgroup's weights are in flight
      plan_one_token(lgk, E, k, sel, rwave, plan, idx_out + (size_t)tok * k, w_out + (size_t)tok * k, true);
      if (inspect) publish_plan_token(tok);
      if (plan_words && (int)threadIdx.x < k)
        store_agent64(planbox + (size_t)tok * k + threadIdx.x,
                      ((uint64_t)tag << 32) | (uint32_t)plan.uexp[threadIdx.x] |
                          (f32_to_bf16(plan.w[0][threadIdx.x]) << 16));
    }
    if (MRMAX == 1 || mult == 1) tile_compute<1, L1, false, kGuChunks>(tl, xr, 1, red, res);
    else if (MRMAX == 2 || mult == 2) tile_compute<(MRMAX >= 2 ? 2 : 1), L1, false, kGuChunks>(tl, xr, mult, red, res);
    else tile_compute<MRMAX, L1, false, kGuChunks>(tl, xr, mult, red, res);
    uint64_t* mine = mbox + (size_t)urow * mrow + ((size_t)slice * t1 + tile) * kGuTileCols;
    for (int m = 0; m < mult; ++m)
#pragma unroll
      for (int h = 0; h < kGuTileCols / kThreads; ++h)
        store_agent64(mine + (size_t)m * mrow + h * kThreads + threadIdx.x,
                      mail_word(res[m * kGuTileCols + h * kThreads + threadIdx.x], tag));
    // the last of the s1 K-slice workgroups of (u, tile) reduces them (it
    // re-arms the counter: every arrival of the launch is in)
    __shared__ int s_last;
    if (threadIdx.x == 0) {
      int* c = cnt_gu + (u * t1 + tile) * kFlagStride;
      const int prev = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == s1 - 1;
      if (prev == s1 - 1) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    // act columns tile*kGuActCols + i: gate and up summed over the slices in
    // slice order (the words of the others may still be in flight: read until
    // tagged; one column per thread), SwiGLU, published as tagged pair words
    const size_t slice_words = (size_t)t1 * kGuTileCols;
    __shared__ float s_sum[kGuTileCols];
    uint64_t* abox = abox_all + (size_t)urow * act_words + (size_t)tile * (kGuActCols / 2);
    for (int m = 0; m < mult; ++m) {
      const uint64_t* box = mbox + ((size_t)urow + m) * mrow + (size_t)tile * kGuTileCols;
#pragma unroll
      for (int h = 0; h < kGuTileCols / kThreads; ++h) {
        const int c = h * kThreads + threadIdx.x;
        s_sum[c] = sum_mail_ordered(box + c, slice_words, s1, tag, kSpinLimit >> 6, err);
      }
      __syncthreads();
      if (threadIdx.x < kGuActCols / 2) {
        const int i = 2 * threadIdx.x;
        const uint32_t a0 = f32_to_bf16(silu_f32(round_bf16(s_sum[i])) * round_bf16(s_sum[kGuActCols + i]));
        const uint32_t a1 = f32_to_bf16(silu_f32(round_bf16(s_sum[i + 1])) * round_bf16(s_sum[kGuActCols + i + 1]));
        const uint32_t pair = a0 | (a1 << 16);
        store_agent64(abox + (size_t)m * act_words + threadIdx.x, ((uint64_t)tag << 32) | pair);
        // one copy of act for inspection
        const int col = tile * kGuActCols + i;
        if (inspect && col < MI) *reinterpret_cast<uint32_t*>(act + ((size_t)u * kMaxTok + m) * MI + col) = pair;
      }
      __syncthreads();
    }
    return;
  }

  // ---- down workgroup (u, tile)
  const int bid = (int)blockIdx.x - n_gu;
  const int u = bid / t2;
  const int tile = bid % t2;
  if (u >= nunique) return;
  // several tokens: expert and routing weight of pair u, published by the
  // token's gate_up writer early in the launch
  uint32_t pword = 0u;
  if (plan_words) wait_mail_block<1>(planbox + u, 0, 1, tag, &pword, err);
  const int e = plan_words ? (int)(pword & 0xffffu) : (fast ? sel_expert(u - tok * k) : plan.uexp[u]);
  const int mult = fast ? 1 : plan.umult[u];
  const int urow = fast ? u : plan.urow[u];
  const int cc = threadIdx.x & (CH2 - 1);
  const int tcol = dn_col0(tile, TC2, H);
  const int col0 = tcol + cc * 32;
  const int colw = col0 < H ? (col0 >> 3) : -1;
  const uint32_t* we = wdn + (size_t)e * MI * (H >> 3);
  const uint16_t* se = sdn + (size_t)e * (MI / gs_dn) * H;
  // this workgroup's weights (first pass): they depend only on the routing
  // and are in by the time the act rows are
  constexpr int L2 = DL;
  TileLoad<L2> tl;
  if (fast && tdn != nullptr && TC2 == kTileCols && L2 == kNarrowR)
    // decode tiles: 256-column tile t of 16-row runs is column tile t of the
    // one-token launch's down tiles
    tile_load_dtile<L2, CH2>(tdn + (size_t)e * MI * (H >> 3), H / kTileCols, tile, kNarrowR, 4 * cc, se, H, gs_dn,
                             0, min(MI, (kThreads / CH2) * L2), colw, tl);
  else
    tile_load<L2, CH2>(we, se, H, gs_dn, 0, min(MI, (kThreads / CH2) * L2), colw, tl);
  // the products need the routing weight of the pair
  if (fast && !plan_words) plan_one_token(lgk, E, k, sel, rwave, plan, idx_out, w_out, false);
  const float w_pair = plan_words ? bf16_to_f32(pword >> 16) : (fast ? plan.w[0][u - tok * k] : 0.f);
  uint64_t* abox = abox_all + (size_t)urow * act_words;

  // all act rows of u (mult x act_words pair words) into LDS
  __shared__ uint32_t s_act[MRMAX][kMaxMI / 2];
  {
    constexpr int kWordsPerThread = MRMAX * (kMaxMI / 2) / kThreads;
    const int nw = mult * (int)act_words;  // words to fetch, word q at (m, w) = (q / act_words, q % act_words)
    uint32_t got[kWordsPerThread];
    // thread t takes words q = t + i * kThreads
    int n_mine = 0;
    while (n_mine < kWordsPerThread && (int)threadIdx.x + n_mine * kThreads < nw) ++n_mine;
    // the words of one thread are kThreads apart in q; q -> mailbox offset is
    // (q / act_words) * act_words + q % act_words == q (rows are contiguous)
    wait_mail_block<kWordsPerThread>(abox + threadIdx.x, kThreads, n_mine, tag, got, err);
#pragma unroll
    for (int i = 0; i < kWordsPerThread; ++i) {
      const int q = threadIdx.x + i * kThreads;
      if (i < n_mine) s_act[q / (int)act_words][q % (int)act_words] = got[i];
    }
    __syncthreads();
  }
  XRows xr;
#pragma unroll
  for (int m = 0; m < kMaxTok; ++m) xr.p[m] = reinterpret_cast<const uint16_t*>(&s_act[min(min(m, mult - 1), MRMAX - 1)][0]);
  float y[MRMAX];
  if (MRMAX == 1 || mult == 1) down_tile<1, L2, CH2>(we, se, H, MI, gs_dn, colw, tl, xr, 1, red, res, y);
  else if (MRMAX == 2 || mult == 2) down_tile<(MRMAX >= 2 ? 2 : 1), L2, CH2>(we, se, H, MI, gs_dn, colw, tl, xr, mult, red, res, y);
  else down_tile<MRMAX, L2, CH2>(we, se, H, MI, gs_dn, colw, tl, xr, mult, red, res, y);

  // weighted products at (token, slot), published for the combiner
  const int col = tcol + threadIdx.x;
  const bool mine = (int)threadIdx.x < TC2 && col < H;
  if (mine) {
#pragma unroll
    for (int m = 0; m < MRMAX; ++m) {
      if (m < mult) {
        const int t = fast ? tok : plan.utok[u][m], j = fast ? u - tok * k : plan.uslot[u][m];
        const float pr = round_bf16(round_bf16(y[m]) * (fast ? w_pair : plan.w[t][j]));
        store_agent64(pbox + ((size_t)t * k + j) * H + col, mail_word(pr, tag));
        if (inspect) prod[((size_t)t * k + j) * H + col] = pr;
      }
    }
  }
  // combiner of this tile: the last unique slot (fast path: the last slot of
  // each token, one combiner per token and tile). Per token, the k products
  // in slot order. The last of the combiners advances the epoch (the count
  // is looked at at the end).
  if (fast ? (u - tok * k != k - 1) : (u != nunique - 1)) return;
  const int ncomb = fast ? B * t2 : t2;
  int comb_prev = 0;
  if (threadIdx.x == 0) comb_prev = __hip_atomic_fetch_add(cnt_rdy, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (mine) {
    for (int t = fast ? tok : 0; t < (fast ? tok + 1 : B); ++t) {
      const float accv = sum_mail_ordered(pbox + (size_t)t * k * H + col, H, k, tag, kSpinLimit >> 6, err);
      float r = round_bf16(accv);
      if (shared != nullptr) {
        const float g = bf16_to_f32(gate[t]);
        const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
        r = round_bf16(r + round_bf16(bf16_to_f32(shared[(size_t)t * H + col]) * sg));
      }
      out[(size_t)t * H + col] = (uint16_t)f32_to_bf16(r);
    }
  }
  if (threadIdx.x == 0 && comb_prev == ncomb - 1) {
    __hip_atomic_store(epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(cnt_rdy, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------- one-token decode on XCD groups
//
// The one-token layer (H a multiple of 256, MI of 128) in one launch whose
// hand-offs stay inside one XCD where they can. Workgroup b runs on XCD
// (b + c) % 8 for a constant c, so blocks with congruent indices share an L2.
//
// Group g = u * t1 + m: routed slot u, act tile m of 128 act columns (t1 =
// MI / 128), pinned to one XCD (xcd_group). A group owns
//  - s1 = H / 128 gate_up workgroups (K-slice s of 128 rows; gate 128 | up
//    128 columns of act tile m). Each stores its 256 fp32 partial columns as
//    tagged words with plain stores, which stay in the XCD's L2;
//  - t2 = H / 256 down workgroups (column tile c of 256 columns over the 128
//    down rows of act tile m). Each reads the group's s1 x 256 partial words,
//    sums them in slice order, applies SwiGLU into LDS, computes its tile and
//    publishes the fp32 partial y_m[256 c .. 256 c + 255] as device-coherent
//    tagged words.
// Combiners (one per 32 output columns) sum the down partials of each slot
// over m in order, round, weight and round (prod = bf16(bf16(y) * w)), and
// sum the k products in slot order (plus the shared merge). The down output
// y = ((P_0 + P_1) + ...) + P_{t1-1} sums 128-row passes in the order the
// separate down launch's passes do, so both launch forms give the same bits.
//
// Block order: the combiners (padded to whole XCD rounds), then all gate_up
// blocks, then all down blocks. A gate_up block waits on nothing, a down
// block only on gate_up blocks, a combiner only on down blocks: the launch
// completes whenever more workgroups fit on the GPU than there are
// combiners.
//
// TILED: the weights come from decode-tile copies (qmoe_decode_tiles_*):
// every workgroup's 128 x 32 words are one contiguous 16 KB block, word
// (p, t) = thread t's p-th row word at p * 256 + t, so each load instruction
// of a workgroup reads 1 KB in one piece instead of 128-byte (down) or
// 64-byte (gate_up) pieces of rows 512 B to 1 KB apart. Same words, same
// arithmetic: the bits do not change.
constexpr int kXcd = 8;
constexpr int kCombCols = 32;  // output columns per combiner

QMOE_DEV void store_local64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits until the n (<= N) words base[off[i]] carry `tag` and leaves them in
// v[i]. Every round re-reads all words not yet seen tagged, issued back to
// back. PIPE keeps two rounds in flight, so a word that lands is seen about
// half a round trip later (at twice the registers). Bounded: a timeout sets
// *err and leaves the untagged words as they are.
template <int N, bool PIPE>
QMOE_DEV void poll_words(const uint64_t* base, const uint32_t* off, int n, uint32_t tag, uint64_t* v, int* err) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = (i < n) ? load_agent64(base + off[i]) : ((uint64_t)tag << 32);
  if constexpr (PIPE) {
    // two rounds in flight, every word reloaded every round (no branches, so
    // each check waits for its own round only); tagged words are kept in v
    uint64_t a[N], b[N];
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] = load_agent64(base + off[min(i, n - 1)]);
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; ++i) b[i] = load_agent64(base + off[min(i, n - 1)]);
    for (int polls = 0;; ++polls) {
      bool ok = true;
#pragma unroll
      for (int i = 0; i < N; ++i) ok = ok && mail_ready(v[i], tag);
      if (ok) return;
      if (polls >= (kSpinLimit >> 6)) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
#pragma unroll
      for (int i = 0; i < N; ++i) v[i] = mail_ready(v[i], tag) ? v[i] : a[i];
#pragma unroll
      for (int i = 0; i < N; ++i) a[i] = load_agent64(base + off[min(i, n - 1)]);
      ok = true;
#pragma unroll
      for (int i = 0; i < N; ++i) ok = ok && mail_ready(v[i], tag);
      if (ok) return;
#pragma unroll
      for (int i = 0; i < N; ++i) v[i] = mail_ready(v[i], tag) ? v[i] : b[i];
#pragma unroll
      for (int i = 0; i < N; ++i) b[i] = load_agent64(base + off[min(i, n - 1)]);
    }
  } else {
    for (int polls = 0;; ++polls) {
      bool ok = true;
#pragma unroll
      for (int i = 0; i < N; ++i) ok = ok && mail_ready(v[i], tag);
      if (ok) return;
      if (polls >= (kSpinLimit >> 6)) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int i = 0; i < N; ++i)
        if (!mail_ready(v[i], tag)) v[i] = load_agent64(base + off[i]);
    }
  }
}

// Group of a block slot: XCD x, j-th group slot of that XCD. With line
// pairs (pr > 0 whole rounds of pairs) the act tiles 2p and 2p + 1 of a slot
// (the two halves of the same 128-byte gate and up lines) share an XCD for
// the first 8 pr pairs; the remaining groups are dealt one per XCD, so every
// XCD holds the same number of groups.
QMOE_DEV int xcd_group(int x, int j, int pr) {
  if (j < 2 * pr) return 2 * (x + kXcd * (j >> 1)) + (j & 1);
  return 2 * kXcd * pr + (j - 2 * pr) * kXcd + x;
}

// One lane polls one word (spaced polls, bounded) until it carries `tag`;
// the workgroup then goes on. Used before a workgroup reads many words
// that land together, so that the wait itself costs one load per poll.
// (Keeping four polls in flight made the gate open sooner but measured
// slower: the reads that follow then more often find a word missing.)
QMOE_DEV void gate_word(const uint64_t* p, uint32_t tag, int* err) {
  if (threadIdx.x == 0) {
    for (int polls = 0; !mail_ready(load_agent64(p), tag); ++polls) {
      if (polls >= (kSpinLimit >> 6)) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

template <int KPL, int GR, bool TILED>
__global__ __launch_bounds__(kThreads, 4) void moe_decode_xcd_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ logits, const uint32_t* __restrict__ wgu,
    const uint16_t* __restrict__ sgu, const uint32_t* __restrict__ wdn, const uint16_t* __restrict__ sdn,
    const uint32_t* __restrict__ tgu, const uint32_t* __restrict__ tdn, const uint16_t* __restrict__ sh_gu,
    const uint16_t* __restrict__ sh_dn, int n_sd, int B,
    int E, int k, int H, int MI, int gs_gu, int gs_dn, int n_groups, int gslots, int pair_rounds,
    DecodePlan* __restrict__ gplan, uint64_t* __restrict__ mbox, uint16_t* __restrict__ act,
    float* __restrict__ prod, int* __restrict__ counters, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ out, int64_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out) {
  uint32_t* epoch = reinterpret_cast<uint32_t*>(counters + kEpochSlot);
  int* err = counters + kErrSlot;
  const uint32_t tag = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  const bool inspect = gplan != nullptr;
  __shared__ float red[kNarrowLanes * kTileCols];
  __shared__ DecodePlan plan;
  const int t1 = MI / kGuActCols, s1 = H / kNarrowRows, t2 = H / kTileCols;
  // gslots group slots per XCD; groups padded to gp = 8 gslots. Blocks:
  // combiners (padded to whole XCD rounds), gate_up, down.
  const int gp = kXcd * gslots;
  const int n_cb = B * (H / kCombCols), n_cbp = ceil_div(n_cb, kXcd) * kXcd;
  const int n_gu = gp * s1, n_dn = gp * t2;
  const int bid = (int)blockIdx.x - n_cbp;
  // mailbox: gate_up partials [gp][s1][256], down partials [gp][H]
  uint64_t* gbox = mbox;
  uint64_t* dbox = gbox + (size_t)gp * s1 * kGuTileCols;

  // role and group of this block
  int role, g = 0, s = 0, c = 0, tok = 0;
  if (bid < 0) {
    role = 2;
    const int b = (int)blockIdx.x, per_tok = H / kCombCols;
    if (b >= n_cb) return;  // padding
    tok = b / per_tok;
    c = b % per_tok;
  } else if (bid < n_gu) {
    role = 0;
    const int i = bid / kXcd;
    g = xcd_group(bid % kXcd, i / s1, pair_rounds);
    s = i % s1;
  } else {
    role = 1;
    const int b = bid - n_gu, i = b / kXcd;
    g = xcd_group(b % kXcd, i / t2, pair_rounds);
    c = i % t2;
  }
  if ((role == 0 || role == 1) && g >= n_groups) return;  // padding
  // the launch epoch advances once the down blocks (when done) and the
  // combiners (once routed) have counted: by then every block of the launch
  // has read it (each gate_up block's words were awaited by a down block).
  // Down blocks count on the counter of their column tile, the last of a
  // tile on the top counter with the combiners.
  auto arrive = [&](int* group_ctr, int group_total) {
    if (threadIdx.x == 0) arrive2(group_ctr, group_total, counters, t2 + n_cb, epoch, tag);
  };
  const int u = g / t1, m = g % t1;
  if (role != 2) tok = u / k;

  // the token's logits (routing wave) and, for gate_up blocks, the
  // activation rows of the slice go out first: neither depends on the
  // routing, and nothing waits for the launch tag before them
  const int rwave = blockIdx.x & 3;
  const bool routes = (int)(threadIdx.x >> 6) == rwave;
  uint4 lraw[KPL / 8];
  if (routes) route_load_vec<KPL>(logits + (size_t)tok * E, E, lraw);
  constexpr int kHalves = kNarrowRows / (kNarrowLanes * GR);  // 1, or 2 for 8 rows per lane
  uint32_t xp[kHalves][GR / 2];
  if (role == 0) {
#pragma unroll
    for (int h = 0; h < kHalves; ++h) {
      const int kh = s * kNarrowRows + h * kNarrowLanes * GR;
      const uint4* xa = reinterpret_cast<const uint4*>(x + (size_t)tok * H + kh + (threadIdx.x / kNarrowChunks) * GR);
#pragma unroll
      for (int i = 0; i < GR / 8; ++i) {
        const uint4 v = xa[i];
        xp[h][4 * i] = v.x; xp[h][4 * i + 1] = v.y; xp[h][4 * i + 2] = v.z; xp[h][4 * i + 3] = v.w;
      }
    }
  }

  // routing of this block's token: one wave selects, the others take the
  // selection from LDS; lane r of sel holds the key of rank r
  // A gate_up or down block needs only the expert of its own slot, fixed
  // after round u % k + 1 of the selection: it takes that many rounds and
  // starts streaming. The token's first gate_up block (which writes the
  // routing outputs) selects all k again once its loads are out; the
  // combiners take all k at once.
  uint32_t sel;
  {
    __shared__ uint32_t s_sel[QMOE_KMAX];
    if (routes) {
      uint32_t key[KPL];
      float lgk[KPL];
      route_keys_vec<KPL>(lraw, E, key, lgk);
      RouteSelect<KPL> rsel;
      rsel.init(key);
      rsel.rounds(0, (role == 2) ? k : u % k + 1);
      sel = rsel.mine;
      if ((threadIdx.x & 63) < QMOE_KMAX) s_sel[threadIdx.x & 63] = sel;
    }
    __syncthreads();
    sel = ((threadIdx.x & 63) < QMOE_KMAX) ? s_sel[threadIdx.x & 63] : 0u;
  }
  // the combiners count as arrived once started (the launch tag, loaded
  // first, is awaited only here, after the routing loads), on the top counter
  if (role == 2) arrive(nullptr, 0);

  if (role == 0) {
    // ---- gate_up slice s of group g
    const int e = route_key_expert(route_sel_rank(sel, u % k));
    const int N = 2 * MI;
    const uint32_t* we = wgu + (size_t)e * H * (N >> 3);
    const uint16_t* se = sgu + (size_t)e * (H / gs_gu) * N;
    const int k0 = s * kNarrowRows;
    NarrowLoad<GR> tl[kHalves];
    if constexpr (TILED) {
      const uint32_t* tb = tgu + (size_t)e * H * (N >> 3) + (size_t)(s * t1 + m) * kDecodeTileWords;
#pragma unroll
      for (int h = 0; h < kHalves; ++h)
        narrow_load_tiled<GR>(tb + h * GR * kThreads, se, N, gs_gu, k0 + h * kNarrowLanes * GR,
                              narrow_gu_colw(threadIdx.x % kNarrowChunks, m, MI), tl[h]);
    } else {
#pragma unroll
      for (int h = 0; h < kHalves; ++h)
        narrow_load<GR>(we, se, N, gs_gu, k0 + h * kNarrowLanes * GR,
                        narrow_gu_colw(threadIdx.x % kNarrowChunks, m, MI), tl[h]);
    }
    if (u % k == 0 && m == 0 && s == 0) {
      // the routing outputs of this token (one workgroup per token), while
      // the weights are in flight: the rest of the selection first
      // (the logits again, from L2: keeping them in registers from the
      // routing on would cost every block the registers)
      float lgk[KPL];
      if (routes) {
        uint4 lr[KPL / 8];
        route_load_vec<KPL>(logits + (size_t)tok * E, E, lr);
        uint32_t key[KPL];
        route_keys_vec<KPL>(lr, E, key, lgk);
        sel = wave_route_select<KPL>(key, k);
      }
      plan_one_token<KPL>(lgk, E, k, sel, rwave, plan, idx_out + (size_t)tok * k, w_out + (size_t)tok * k, true);
      if (inspect && (int)threadIdx.x < k) {
        const int uu = tok * k + threadIdx.x;
        gplan->uexp[uu] = plan.uexp[threadIdx.x];
        gplan->umult[uu] = 1;
        gplan->utok[uu][0] = tok;
        gplan->uslot[uu][0] = threadIdx.x;
        gplan->urow[uu] = uu;
        gplan->w[tok][threadIdx.x] = plan.w[0][threadIdx.x];
      }
      if (inspect && tok == 0 && threadIdx.x == 0) gplan->nunique = B * k;
    }
    float own = 0.f;
#pragma unroll
    for (int h = 0; h < kHalves; ++h) own += narrow_compute<GR>(tl[h], xp[h], red);
    store_local64(gbox + ((size_t)g * s1 + s) * kGuTileCols + threadIdx.x, mail_word(own, tag));
    return;
  }

  if (role == 1) {
    // ---- down rows [128 m, 128 m + 128) x columns [256 c, 256 c + 256) of
    // group g: narrow tile of 8 row-lanes x 16 rows
    constexpr int R = kNarrowR;
    static_assert(kNarrowRows == kGuActCols, "one down pass covers one act tile");
    const int e = route_key_expert(route_sel_rank(sel, u % k));
    const int colw = c * (kTileCols / 8) + (int)(threadIdx.x % kNarrowChunks);
    const uint32_t* we = wdn + (size_t)e * MI * (H >> 3);
    const uint16_t* se = sdn + (size_t)e * (MI / gs_dn) * H;
    NarrowPairs<R> up;
    {
      NarrowLoad<R> tl;
      if constexpr (TILED)
        narrow_load_tiled<R>(tdn + (size_t)e * MI * (H >> 3) + (size_t)(m * t2 + c) * kDecodeTileWords, se, H, gs_dn,
                             m * kGuActCols, colw, tl);
      else
        narrow_load<R>(we, se, H, gs_dn, m * kGuActCols, colw, tl);
      narrow_unpack<R>(tl, up);  // while the act rows are on their way
      // keep the unpacked pairs ahead of the wait (the compiler would
      // otherwise sink the unpack below it, onto the path after the act)
#pragma unroll
      for (int i = 0; i < R / 2; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(up.p[i][j])::"memory");
    }
    // the group's act tile from the gate_up partials (same XCD): column
    // threadIdx.x (gate 0..127 | up 128..255) summed over the slices in
    // slice order, then SwiGLU into LDS
    __shared__ float s_sum[kGuTileCols];
    __shared__ uint32_t s_act[kGuActCols / 2];
    {
      const uint64_t* gw = gbox + (size_t)g * s1 * kGuTileCols + threadIdx.x;
      float sum = 0.f;
      // batches of 8 words (4 beside 16 logits per lane): the unpacked
      // weights hold 64 registers
      constexpr int kPoll = KPL <= 8 ? 8 : 4;
      for (int s0 = 0; s0 < s1; s0 += kPoll) {
        uint32_t off[kPoll];
        uint64_t v[kPoll];
#pragma unroll
        for (int i = 0; i < kPoll; ++i) off[i] = (uint32_t)(min(s0 + i, s1 - 1) * kGuTileCols);
        poll_words<kPoll, false>(gw, off, min(kPoll, s1 - s0), tag, v, err);
#pragma unroll
        for (int i = 0; i < kPoll; ++i)
          if (s0 + i < s1) sum += mail_value(v[i]);
      }
      s_sum[threadIdx.x] = sum;
      __syncthreads();
      if (threadIdx.x < kGuActCols / 2) {
        const int i = 2 * threadIdx.x;
        const uint32_t a0 = f32_to_bf16(silu_f32(round_bf16(s_sum[i])) * round_bf16(s_sum[kGuActCols + i]));
        const uint32_t a1 = f32_to_bf16(silu_f32(round_bf16(s_sum[i + 1])) * round_bf16(s_sum[kGuActCols + i + 1]));
        const uint32_t pair = a0 | (a1 << 16);
        s_act[threadIdx.x] = pair;
        if (inspect && c == 0) *reinterpret_cast<uint32_t*>(act + (size_t)u * kMaxTok * MI + m * kGuActCols + i) = pair;
      }
      __syncthreads();
    }
    // act pairs of the row-lane's 16 rows
    const int r = threadIdx.x / kNarrowChunks;
    uint32_t xp[R / 2];
#pragma unroll
    for (int i = 0; i < R / 2; ++i) xp[i] = s_act[(R / 2) * r + i];
    const float y = narrow_dots<R>(up, xp, red);
    store_agent64(dbox + (size_t)g * H + c * kTileCols + threadIdx.x, mail_word(y, tag));
    arrive(counters + kFlagStride * (1 + c), n_groups);
    return;
  }

  // ---- combiner of token tok, columns [32 c, 32 c + 32): thread (q, lane)
  // forms the products of slots q, q + 8 at column lane; the first 32
  // threads sum them in slot order
  {
    float lgk[KPL];
    if (routes) {
      uint4 lr[KPL / 8];
      route_load_vec<KPL>(logits + (size_t)tok * E, E, lr);
      uint32_t key[KPL];
      route_keys_vec<KPL>(lr, E, key, lgk);
    }
    plan_one_token<KPL>(lgk, E, k, sel, rwave, plan, idx_out, w_out, false);
  }
  // With the shared expert in the launch (n_sd, one token): this combiner's
  // 32 columns of sh = bf16(act . W_sd[n, :]), act = bf16(bf16(silu(g)) * u)
  // from the projection row sh_gu (gate | up), in the arithmetic of the
  // separate shared-down GEMV (qmoe_bf16_gemv_swiglu): lane l takes the act
  // pieces 8 (l + 64 i), i < ppl, each row one wave sum. Wave w computes rows
  // 32 c + 8 w .. + 7 while the products are still on their way.
  __shared__ float s_sh[kCombCols];
  if (n_sd > 0) {
    const int wl = threadIdx.x & 63, wv_ = (int)(threadIdx.x >> 6);
    const int pieces = ceil_div(MI, 8);
    const int ppl = pieces <= 64 ? 1 : pieces <= 128 ? 2 : 4;  // MI <= 2048 (xcd_shape)
    auto rows = [&](auto ppl_c) {
      constexpr int PPL = decltype(ppl_c)::value, RB = 8 / PPL;  // rows per batch: 8 weight pieces per lane
      uint4 av[PPL];
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        const int kk = 8 * (wl + 64 * i);
        uint4 a = make_uint4(0u, 0u, 0u, 0u);
        if (kk < MI) {
          const uint4 gg = *reinterpret_cast<const uint4*>(sh_gu + kk);
          const uint4 uu = *reinterpret_cast<const uint4*>(sh_gu + MI + kk);
          const uint32_t gw[4] = {gg.x, gg.y, gg.z, gg.w}, uw[4] = {uu.x, uu.y, uu.z, uu.w};
          uint32_t o[4];
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
            o[qq] = swiglu_bf16_bits(gw[qq] & 0xffffu, uw[qq] & 0xffffu) | (swiglu_bf16_bits(gw[qq] >> 16, uw[qq] >> 16) << 16);
          a = make_uint4(o[0], o[1], o[2], o[3]);
        }
        av[i] = a;
      }
#pragma unroll 1
      for (int b = 0; b < 8; b += RB) {
        uint4 wq[RB][PPL];
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
          for (int i = 0; i < PPL; ++i) {
            const int kk = 8 * (wl + 64 * i), n = c * kCombCols + 8 * wv_ + b + r;
            wq[r][i] = (kk < MI && n < H) ? *reinterpret_cast<const uint4*>(sh_dn + (size_t)n * MI + kk)
                                          : make_uint4(0u, 0u, 0u, 0u);
          }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < PPL; ++i) {
            const uint4 w4 = wq[r][i], a4 = av[i];
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4.x), __builtin_bit_cast(bf16x2_t, a4.x), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4.y), __builtin_bit_cast(bf16x2_t, a4.y), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4.z), __builtin_bit_cast(bf16x2_t, a4.z), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4.w), __builtin_bit_cast(bf16x2_t, a4.w), acc, false);
          }
          const float sum = wave_sum_f32(acc);
          if (wl == 0) s_sh[8 * wv_ + b + r] = round_bf16(sum);
        }
      }
    };
    if (ppl == 1) rows(IntConst<1>{});
    else if (ppl == 2) rows(IntConst<2>{});
    else rows(IntConst<4>{});
  }
  __shared__ float s_pr[QMOE_KMAX][kCombCols];
  const int q = threadIdx.x / kCombCols, lane = threadIdx.x % kCombCols;
  const int col = c * kCombCols + lane;
  constexpr int kSlotLanes = kThreads / kCombCols;  // 8
  const int nj = (k - q + kSlotLanes - 1) / kSlotLanes;  // slots of this thread
  const int nw = nj * t1;                                // words: (slot jj, tile mm) in order
  const uint64_t* cbase = dbox + (size_t)tok * k * t1 * H + col;
  // the routing weights of this thread's slots (q, q + 8; k <= 16)
  static_assert(QMOE_KMAX <= 2 * kSlotLanes, "two slots per combiner thread");
  const float w_lo = plan.w[0][q], w_hi = (q + kSlotLanes < k) ? plan.w[0][q + kSlotLanes] : 0.f;
  // the down partials land over a few microseconds: one lane waits on the
  // last word of slot min(k, 8) - 1 (the last slot that every thread reads
  // first), then every thread reads its words; threads that also hold a
  // slot >= 8 keep polling those, which land later. Measured against gating
  // on the last slot's word (0.35 us later), on every group's word (all, or
  // all but an eighth) and against no gate: this one ends soonest.
  gate_word(dbox + (size_t)(tok * k * t1 + min(k, kSlotLanes) * t1 - 1) * H + c * kCombCols, tag, err);
  float run = 0.f;
  // word (slot q + 8 jj, act tile mm) of the next batch, stepped without
  // divisions (the offsets are per thread, so divisions would be vector code)
  int jj = 0, mm = 0;
  for (int w0 = 0; w0 < nw; w0 += 8) {
    uint32_t off[8];
    uint64_t v[8];
    {
      int ja = jj, ma = mm;
      uint32_t o = (uint32_t)(((q + kSlotLanes * ja) * t1 + ma) * H);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        off[i] = o;  // past the last word: repeats it (not read)
        if (w0 + i + 1 < nw) {
          ++ma;
          o += (uint32_t)H;
          if (ma == t1) {
            ma = 0;
            ++ja;
            o += (uint32_t)((kSlotLanes - 1) * t1 * H);
          }
        }
      }
    }
    poll_words<8, false>(cbase, off, min(8, nw - w0), tag, v, err);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (w0 + i < nw) {
        run = (mm == 0) ? mail_value(v[i]) : run + mail_value(v[i]);
        if (mm == t1 - 1) {
          const int j = q + kSlotLanes * jj;
          const float pr = round_bf16(round_bf16(run) * (jj == 0 ? w_lo : w_hi));
          s_pr[j][lane] = pr;
          if (inspect) prod[((size_t)tok * k + j) * H + col] = pr;
          mm = 0;
          ++jj;
        } else {
          ++mm;
        }
      }
    }
  }
  __syncthreads();
  if (q == 0) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) acc += s_pr[j][lane];
    float rr = round_bf16(acc);
    if (shared != nullptr || n_sd > 0) {
      const float gg = bf16_to_f32(gate[tok]);
      const float sg = round_bf16(1.0f / (1.0f + expf(-gg)));
      // the shared row: this combiner's own (s_sh, written before the
      // barrier above) or the given one
      const float shv = (n_sd > 0) ? s_sh[lane] : bf16_to_f32(shared[(size_t)tok * H + col]);
      rr = round_bf16(rr + round_bf16(shv * sg));
    }
    out[(size_t)tok * H + col] = (uint16_t)f32_to_bf16(rr);
  }
}

// ---------------------------------------------------------------- standalone GEMM (M <= 4)
//
// Split-K over a grid (column tile, K-slice). Every slice but the last stores
// its fp32 partial columns as tagged words in the counters array's mailbox;
// the last slice (the highest block indices, so it waits only on workgroups
// dispatched before it) keeps its own partial in LDS, reads the others' in
// slice order as soon as they carry this launch's tag, adds its own last and
// rounds. No arrival counter and no wait for store completion sits between
// the partials and the result. The tag is the decode epoch of the same
// counters array (tags keep growing across both kinds of launch, so no word of
// an earlier launch of either is ever taken); the last of the reducing
// workgroups to finish advances it.
template <int MR, int L>
__global__ __launch_bounds__(kThreads) void w4a16_gemv_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
    uint16_t* __restrict__ y, int M, int K, int N, int gs, int* __restrict__ counters) {
  uint32_t* epoch = reinterpret_cast<uint32_t*>(counters + kEpochSlot);
  const uint32_t tag = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[MR * kTileCols];
  const int ntile = blockIdx.x, ntiles = gridDim.x;
  const int slice = blockIdx.y;
  const int nslices = gridDim.y;
  const int ks = kRowLanes * L;
  const int k0 = slice * ks;
  const int kend = min(K, k0 + ks);
  const int cc = threadIdx.x & (kChunks - 1);
  const int col0 = ntile * kTileCols + cc * 32;
  const int colw = col0 < N ? (col0 >> 3) : -1;
  XRows xr;
#pragma unroll
  for (int m = 0; m < 4; ++m) xr.p[m] = x + (size_t)min(m, M - 1) * K;
  TileLoad<L> tl;
  tile_load<L>(w, s, N, gs, k0, kend, colw, tl);
  tile_compute<MR, L, false>(tl, xr, M, red, res);

  // mailbox words [ntile][slice < nslices - 1][MR][256]
  uint64_t* mbox = reinterpret_cast<uint64_t*>(counters + kMailboxBase) +
                   (size_t)ntile * (nslices - 1) * MR * kTileCols;
  const int col = ntile * kTileCols + threadIdx.x;
  if (slice != nslices - 1) {
    for (int m = 0; m < M; ++m)
      store_agent64(mbox + ((size_t)slice * MR + m) * kTileCols + threadIdx.x,
                    mail_word(res[m * kTileCols + threadIdx.x], tag));
    return;
  }
  int* err = counters + kErrSlot;
  for (int m = 0; m < M; ++m) {
    const float sum = sum_mail_ordered(mbox + (size_t)m * kTileCols + threadIdx.x, (size_t)MR * kTileCols,
                                       nslices - 1, tag, kSpinLimit >> 6, err) + res[m * kTileCols + threadIdx.x];
    if (col < N) y[(size_t)m * N + col] = (uint16_t)f32_to_bf16(sum);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int* cnt = counters;
    if (__hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ntiles - 1) {
      __hip_atomic_store(epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// One-row GEMV on narrow tiles (M = 1): workgroup (column tile of 256,
// K-slice of 8 RR rows), thread = (row-lane of RR rows, chunk of 8 columns).
// 128-row slices (256 workgroups for 2048 x 4096) measured fastest with the
// weights read nontemporally; every slice adds partial words the reducer
// waits for, so 64-row ones lose again.
// The slices of a column tile share an XCD when the tile count is a
// multiple of 8 (block (tile, slice) runs on XCD (slice * ntiles + tile) % 8):
// their partials then stay in that XCD's L2 (LOCAL). The last slice keeps
// its own partial, waits for the others' tagged words (all outstanding ones
// re-read together), adds them in slice order and its own last. The launch
// epoch advances on the last arrival of the other slices (when stored) and
// the reducers (when started), off the reducers' path.
template <bool LOCAL, int RR>
__global__ __launch_bounds__(kThreads) void w4a16_gemv_narrow_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
    uint16_t* __restrict__ y, int K, int N, int gs, int* __restrict__ counters) {
  uint32_t* epoch = reinterpret_cast<uint32_t*>(counters + kEpochSlot);
  int* err = counters + kErrSlot;
  const uint32_t tag = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  __shared__ float red[kNarrowLanes * kTileCols];
  const int tile = blockIdx.x, ntiles = gridDim.x, slice = blockIdx.y, nslices = gridDim.y;
  const bool reducer = slice == nslices - 1;
  // every workgroup counts on its tile's counter, the last of a tile on the
  // top one; the last tile advances the epoch
  auto arrive = [&]() {
    if (threadIdx.x == 0) arrive2(counters + kFlagStride * (1 + tile), nslices, counters, ntiles, epoch, tag);
  };
  const int k0 = slice * (kNarrowLanes * RR);
  const int colw = tile * (kTileCols / 8) + (int)(threadIdx.x % kNarrowChunks);
  uint32_t xp[RR / 2];
  {
    const uint4* xa = reinterpret_cast<const uint4*>(x + k0 + (threadIdx.x / kNarrowChunks) * RR);
#pragma unroll
    for (int i = 0; i < RR / 8; ++i) {
      const uint4 v = xa[i];
      xp[4 * i] = v.x; xp[4 * i + 1] = v.y; xp[4 * i + 2] = v.z; xp[4 * i + 3] = v.w;
    }
  }
  NarrowLoad<RR> tl;
  narrow_load<RR>(w, s, N, gs, k0, colw, tl);
  // the reducer counts as arrived once its loads are out (the launch tag,
  // loaded first, is not awaited before them)
  if (reducer) arrive();
  const float own = narrow_compute<RR>(tl, xp, red);
  // mailbox words [tile][slice < nslices - 1][256]
  uint64_t* gw = reinterpret_cast<uint64_t*>(counters + kMailboxBase) +
                 (size_t)tile * (nslices - 1) * kTileCols + threadIdx.x;
  if (!reducer) {
    if (LOCAL) store_local64(gw + (size_t)slice * kTileCols, mail_word(own, tag));
    else store_agent64(gw + (size_t)slice * kTileCols, mail_word(own, tag));
    arrive();
    return;
  }
  float sum = 0.f;
  for (int s0 = 0; s0 < nslices - 1; s0 += 16) {
    uint32_t off[16];
    uint64_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) off[i] = (uint32_t)(min(s0 + i, nslices - 2) * kTileCols);
    poll_words<16, false>(gw, off, min(16, nslices - 1 - s0), tag, v, err);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (s0 + i < nslices - 1) sum += mail_value(v[i]);
  }
  y[(size_t)tile * kTileCols + threadIdx.x] = (uint16_t)f32_to_bf16(sum + own);
}

}  // namespace

// ---------------------------------------------------------------- no-allocation scratch
//
// Counters array of qmoe_moe_decode_noalloc: arrival counters, epoch, error
// flag and mailbox in one fixed device array per GPU, held until the process
// ends. The loader zero-fills it; the first call on a device (outside graph
// capture) also clears it in stream order.
constexpr size_t kScratchBytes = (size_t)8 << 20;
constexpr int kScratchInts = (int)(kScratchBytes / sizeof(int));
static __device__ __align__(256) int scratch[kScratchInts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device (nullptr: not looked up yet)

__global__ __launch_bounds__(256) void clear_ints_kernel(int* __restrict__ p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

// Address of the current device's scratch (looked up once per device with
// that device current), or nullptr with *rc set.
static int* device_scratch(hipStream_t stream, int* rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *rc = e != hipSuccess ? (int)e : QMOE_EINVAL;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    int* p = nullptr;
    e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *rc = e != hipSuccess ? (int)e : QMOE_EINVAL;
      return nullptr;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone) {
      hipLaunchKernelGGL(clear_ints_kernel, dim3(1024), dim3(256), 0, stream, p, kScratchInts);
      e = hipGetLastError();
      if (e != hipSuccess) {
        *rc = (int)e;
        return nullptr;
      }
    }
    g_scratch_ptr[dev] = p;
  }
  *rc = QMOE_OK;
  return g_scratch_ptr[dev];
}

// ---------------------------------------------------------------- workgroup placement
//
// The one-token decode launch (gate_up partials) and the one-row GEMV (slice
// partials) hand data from workgroup to workgroup with workgroup-scope
// stores, which stay in the writing XCD's L2. That is correct only while
// workgroup b runs on XCD (b + c) mod 8 for one c per launch. It is checked
// once per device: every workgroup of a probe grid records its XCC_ID and the
// host tests the congruence. A device that fails it (another XCD count, a
// partition mode, a CU mask), one not yet probed while its stream is being
// captured (the probe synchronises), or one the caller switched off, gets the
// device-coherent forms of those launches instead.
constexpr int kProbeBlocks = 2048;
static __device__ __align__(256) int xcc_seen[kProbeBlocks];
enum : int { kPlaceUnknown = 0, kPlaceOk = 1, kPlaceOther = 2 };
std::mutex g_place_mutex;
int g_place[kMaxDevices];

__global__ __launch_bounds__(kThreads) void xcc_probe_kernel(int* __restrict__ seen) {
  // hardware register XCC_ID (id 20), bits 3:0
  if (threadIdx.x == 0) seen[blockIdx.x] = (int)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15u);
}

static bool xcd_placement(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_place_mutex);
  if (g_place[dev] != kPlaceUnknown) return g_place[dev] == kPlaceOk;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return false;
  int* seen = nullptr;
  if (hipGetSymbolAddress((void**)&seen, HIP_SYMBOL(xcc_seen)) != hipSuccess || seen == nullptr) return false;
  static int host[kProbeBlocks];  // guarded by g_place_mutex
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(kProbeBlocks), dim3(kThreads), 0, stream, seen);
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(host, seen, sizeof(host), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return false;
  const int c = ((host[0] % kXcd) + kXcd) % kXcd;
  bool ok = true;
  for (int b = 0; b < kProbeBlocks && ok; ++b) ok = host[b] == (b + c) % kXcd;
  g_place[dev] = ok ? kPlaceOk : kPlaceOther;
  return ok;
}

// ============================================================================ C ABI

extern "C" {

constexpr int kGemvL = 4;  // rows per lane: 128-row K-slices

// The GEMV keeps its partials in the counters array's mailbox: no workspace.
size_t qmoe_w4a16_gemm_workspace(int M, int K, int N) {
  (void)M; (void)K; (void)N;
  return 0;
}

// Counter slots needed by qmoe_w4a16_gemv (int32, zero on first use): the
// epoch and flag below the mailbox, then [ntiles][nslices - 1][4][256]
// tagged 64-bit words.
int qmoe_w4a16_gemm_counters(int M, int K, int N) {
  (void)M;
  const size_t words = (size_t)host_ceil_div(N, kTileCols) * (host_ceil_div(K, kRowLanes * kGemvL) - 1) * 4 * kTileCols;
  const size_t total = (size_t)kMailboxBase + 2 * words;
  return total > 0x7fffffff ? -1 : (int)total;
}

int qmoe_w4a16_gemv(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                    int group_size, void* workspace, size_t workspace_bytes, void* counters,
                    void* stream) {
  (void)workspace; (void)workspace_bytes;
  if (M < 1 || M > 4 || K < 8 || N < 32 || (N % 32) || (K % 8) || group_size < 8 ||
      (group_size % 8) || (K % group_size) || counters == nullptr || qmoe_w4a16_gemm_counters(M, K, N) < 0)
    return QMOE_EINVAL;
  constexpr int L = kGemvL;
  const int nslices = host_ceil_div(K, kRowLanes * L);
  dim3 grid(host_ceil_div(N, kTileCols), nslices);
  hipStream_t st = (hipStream_t)stream;
  auto* xp = (const uint16_t*)x;
  auto* wp = (const uint32_t*)w;
  auto* sp = (const uint16_t*)scale;
  auto* yp = (uint16_t*)y;
  auto* cnt = (int*)counters;
  if (M == 1 && (N % kTileCols) == 0 && N / kTileCols < kEpochSlot / kFlagStride - 1 && (K % kNarrowRows) == 0 &&
      (group_size % kNarrowR) == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)scale & 15) == 0) {
    // one row: narrow tiles over 128-row slices (2048 x 4096: 256
    // workgroups; with the weights read nontemporally these measured 4.14
    // against 4.72 us for 256-row slices and 5.04 for 64-row ones)
    auto go = [&](auto kl, auto kn, int r) {
      const dim3 g1(N / kTileCols, K / (kNarrowLanes * r));
      if (g1.x % kXcd == 0 && xcd_placement(st))
        hipLaunchKernelGGL(kl, g1, dim3(kThreads), 0, st, xp, wp, sp, yp, K, N, group_size, cnt);
      else hipLaunchKernelGGL(kn, g1, dim3(kThreads), 0, st, xp, wp, sp, yp, K, N, group_size, cnt);
    };
    go(w4a16_gemv_narrow_kernel<true, 16>, w4a16_gemv_narrow_kernel<false, 16>, 16);
  } else if (M == 1) hipLaunchKernelGGL((w4a16_gemv_kernel<1, L>), grid, dim3(kThreads), 0, st, xp, wp, sp, yp, M, K, N, group_size, cnt);
  else if (M == 2) hipLaunchKernelGGL((w4a16_gemv_kernel<2, L>), grid, dim3(kThreads), 0, st, xp, wp, sp, yp, M, K, N, group_size, cnt);
  else hipLaunchKernelGGL((w4a16_gemv_kernel<4, L>), grid, dim3(kThreads), 0, st, xp, wp, sp, yp, M, K, N, group_size, cnt);
  return (int)hipGetLastError();
}

// Down column tiles of B tokens (either launch form).
static int dn_t2(int B, int H) {
  const int mr = dn_mr_of(B);
  return host_ceil_div(H, mr == 1 ? dn_tile_cols<1>() : (mr == 2 ? dn_tile_cols<2>() : dn_tile_cols<4>()));
}

// Fused launch: gate_up tiles of 256 act columns and its K-slices.
static int fused_t1(int MI) { return host_ceil_div(MI, kGuActCols); }
static int fused_s1(int H) { return host_ceil_div(H, kGuRowLanes * kGuL); }
// The one-token launch on XCD groups takes H a multiple of 256 and MI of 128.
static bool xcd_shape(int B, int H, int MI) { return B == 1 && (H % kTileCols) == 0 && (MI % kGuActCols) == 0; }
// K-slices of the separate gate_up launch: the 128-row narrow slices of the
// one-token XCD-group launch on its shapes, else fused_s1.
static int separate_s1(int B, int H, int MI) { return xcd_shape(B, H, MI) ? H / kNarrowRows : fused_s1(H); }

// Workspace layout of qmoe_moe_decode (byte offsets), shared with the host.
// part1 holds the separate launch's gate_up partials; act and prod are the
// SwiGLU rows and weighted products, kept for inspection.
static void decode_layout(int B, int k, int H, int MI, size_t* off_plan, size_t* off_part1,
                          size_t* off_act, size_t* off_prod, size_t* total) {
  const int umax = B * k;
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o += (bytes + 255) & ~(size_t)255; return at; };
  *off_plan = take(sizeof(DecodePlan));
  *off_part1 = take((size_t)umax * separate_s1(B, H, MI) * kMaxTok * fused_t1(MI) * kGuTileCols * sizeof(float));
  *off_act = take((size_t)umax * kMaxTok * MI * sizeof(uint16_t));
  *off_prod = take((size_t)B * k * H * sizeof(float));
  *total = o;
}

size_t qmoe_moe_decode_workspace(int B, int k, int H, int MI) {
  size_t a, b, c, d, total;
  decode_layout(B, k, H, MI, &a, &b, &c, &d, &total);
  return total;
}

int qmoe_moe_decode_layout(int B, int k, int H, int MI, size_t* off_plan, size_t* off_act, size_t* off_prod) {
  if (B < 1 || B > kMaxTok || k < 1 || k > QMOE_KMAX || H < 1 || MI < 1) return QMOE_EINVAL;
  size_t part1, total;
  decode_layout(B, k, H, MI, off_plan, &part1, off_act, off_prod, &total);
  return QMOE_OK;
}

// Mailbox words (uint64) of the fused launch: gate_up partials, act pairs
// (64 per gate_up tile of 128 act rows), weighted products.
static size_t decode_mail_words(int B, int k, int H, int MI) {
  return (size_t)B * k *
         ((size_t)fused_s1(H) * fused_t1(MI) * kGuTileCols + (size_t)fused_t1(MI) * (kGuActCols / 2) + (size_t)H + 1);
}

// The one-token launch on XCD groups takes H a multiple of 256 and MI of 128.

// Group slots per XCD of the XCD-group launch: with line pairs (an even
// number of act tiles) the act tiles 2p, 2p + 1 of a slot share an XCD.
static int xcd_pair_rounds(int B, int k, int MI) {
  const int t1 = MI / kGuActCols;
  return (t1 % 2) != 0 ? 0 : (B * k * t1 / 2) / kXcd;
}
static int xcd_gslots(int B, int k, int MI) {
  const int ng = B * k * (MI / kGuActCols), pr = xcd_pair_rounds(B, k, MI);
  return 2 * pr + host_ceil_div(ng - 2 * kXcd * pr, kXcd);
}

// Mailbox words of the XCD-group launch: the gate_up partials of every
// K-slice and the down partials, per group slot, then the shared expert's
// output row when the launch computes it.
static size_t xcd_mail_words(int B, int k, int H, int MI) {
  const int s1 = H / kNarrowRows;
  const size_t gp = (size_t)kXcd * xcd_gslots(B, k, MI);
  return gp * ((size_t)s1 * kGuTileCols + (size_t)H) + (size_t)H;
}

int qmoe_moe_decode_counters(int B, int k, int H, int MI) {
  const int umax = B * k;
  const int t1 = fused_t1(MI), t2 = dn_t2(B, H);
  // the two separate launches: cnt_gu | cnt_out; the fused launch: cnt_rdy,
  // then its cnt_gu 128 bytes apart; the epoch and the error flag at
  // kMailboxBase - 2 and - 1; then the fused launch's mailbox
  const int separate = umax * t1 + t2, fused = kFlagStride * (1 + umax * t1);
  if (std::max(separate, fused) > kEpochSlot) return -1;
  size_t words = decode_mail_words(B, k, H, MI);
  if (xcd_shape(B, H, MI)) words = std::max(words, xcd_mail_words(B, k, H, MI));
  const size_t total = (size_t)kMailboxBase + 2 * words;
  return total > 0x7fffffff ? -1 : (int)total;
}

static int decode_check(int B, int E, int k, int H, int MI, int gs_gu, int gs_dn) {
  if (B < 1 || B > kMaxTok || k < 1 || k > QMOE_KMAX || E < k || E > 1024 || H < 32 || (H % 32) ||
      H > 8192 || MI < 32 || (MI % 32) || MI > kMaxMI || gs_gu < 8 || (gs_gu % 8) || (H % gs_gu) ||
      gs_dn < 16 || (gs_dn % 16) || (MI % gs_dn))
    return QMOE_EINVAL;
  return QMOE_OK;
}

int qmoe_moe_decode_gate_up(const void* x, const void* logits, const void* gu_w, const void* gu_s, void* idx_out,
                            void* w_out, int B, int E, int k, int H, int MI, int gs_gu, void* workspace,
                            size_t workspace_bytes, void* counters, void* stream) {
  if (decode_check(B, E, k, H, MI, gs_gu, 32) != QMOE_OK) return QMOE_EINVAL;
  size_t o_plan, o_part1, o_act, o_prod, total;
  decode_layout(B, k, H, MI, &o_plan, &o_part1, &o_act, &o_prod, &total);
  if (workspace_bytes < total) return QMOE_EWORKSPACE;
  char* ws = (char*)workspace;
  const int umax = B * k;
  const int t1 = fused_t1(MI), s1 = separate_s1(B, H, MI);
  hipLaunchKernelGGL((moe_decode_gate_up_kernel<kGuL>), dim3(t1 * s1, umax), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)logits, (const uint32_t*)gu_w, (const uint16_t*)gu_s,
                     B, E, k, H, MI, gs_gu, (DecodePlan*)(ws + o_plan), (float*)(ws + o_part1),
                     (uint16_t*)(ws + o_act), (int*)counters, (int64_t*)idx_out, (uint16_t*)w_out);
  return (int)hipGetLastError();
}

int qmoe_moe_decode_down(const void* dn_w, const void* dn_s, const void* shared, const void* gate, void* out, int B,
                         int k, int H, int MI, int gs_dn, void* workspace, size_t workspace_bytes, void* counters,
                         void* stream) {
  if (decode_check(B, k, k, H, MI, 32, gs_dn) != QMOE_OK || (shared == nullptr) != (gate == nullptr))
    return QMOE_EINVAL;
  size_t o_plan, o_part1, o_act, o_prod, total;
  decode_layout(B, k, H, MI, &o_plan, &o_part1, &o_act, &o_prod, &total);
  if (workspace_bytes < total) return QMOE_EWORKSPACE;
  char* ws = (char*)workspace;
  const int umax = B * k;
  const int t1 = fused_t1(MI), t2 = dn_t2(B, H);
  int* cnt_out = (int*)counters + umax * t1;
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(t2, umax), dim3(kThreads), 0, (hipStream_t)stream, (const uint32_t*)dn_w,
                       (const uint16_t*)dn_s, B, k, H, MI, gs_dn, (const DecodePlan*)(ws + o_plan),
                       (const uint16_t*)(ws + o_act), (float*)(ws + o_prod), cnt_out, (const uint16_t*)shared,
                       (const uint16_t*)gate, (uint16_t*)out);
  };
  if (dn_mr_of(B) == 1) launch(moe_decode_down_kernel<1>);
  else if (dn_mr_of(B) == 2) launch(moe_decode_down_kernel<2>);
  else launch(moe_decode_down_kernel<4>);
  return (int)hipGetLastError();
}

// Decode tiles of one projection's experts, the weight layout of the TILED
// one-token launch: tile b of expert e holds at p * 256 + t the word that
// thread t of the workgroup owning the tile loads as its p-th row word.
//   gate_up (w [E, H, 2 MI / 8], mode 0): tile b = s * t1 + m (K-slice s of
//   128 rows, act tile m); p = h * GR + i reads row 128 s + h * 8 GR +
//   (t / 32) * GR + i, word narrow_gu_colw(t % 32, m, MI);
//   down (w [E, MI, H / 8], mode 1): tile b = m * t2 + c; row 128 m +
//   (t / 32) * 16 + p, word 32 c + t % 32.
// One workgroup per tile: every p reads two 128-byte row pieces per wave
// and writes 1 KB in one piece.
__global__ __launch_bounds__(kThreads) void decode_tiles_kernel(const uint32_t* __restrict__ w, uint32_t* __restrict__ t,
                                                                int rows, int nw, int mode, int gr, int MI, int per) {
  const int e = blockIdx.y, b = blockIdx.x, ntiles = gridDim.x;
  const int tid = threadIdx.x, lane_r = tid / kNarrowChunks, cc = tid % kNarrowChunks;
  const uint32_t* we = w + (size_t)e * rows * nw;
  uint32_t* te = t + ((size_t)e * ntiles + b) * kDecodeTileWords;
  const int q = b / per, r = b % per;  // gate_up: (slice, act tile); down: (act tile, column tile)
#pragma unroll 4
  for (int p = 0; p < kNarrowR; ++p) {
    int row, col;
    if (mode == 0) {
      const int h = p / gr, i = p % gr;
      row = kNarrowRows * q + h * kNarrowLanes * gr + lane_r * gr + i;
      col = narrow_gu_colw(cc, r, MI);
    } else {
      row = kNarrowRows * q + lane_r * kNarrowR + p;
      col = kNarrowChunks * r + cc;
    }
    te[p * kThreads + tid] = we[(size_t)row * nw + col];
  }
}

// The fused launch. ws == nullptr: no inspection copies (the production
// form, which needs no workspace at all).
static int decode_fused_launch(const void* x, const void* logits, const void* gu_w, const void* gu_s,
                               const void* dn_w, const void* dn_s, const void* gu_t, const void* dn_t,
                               const void* shared, const void* gate, void* out, void* idx_out, void* w_out, int B,
                               int E, int k, int H, int MI, int gs_gu, int gs_dn, char* ws, int* counters,
                               hipStream_t stream, const void* sh_gu = nullptr, const void* sh_dn = nullptr) {
  size_t o_plan, o_part1, o_act, o_prod, total;
  decode_layout(B, k, H, MI, &o_plan, &o_part1, &o_act, &o_prod, &total);
  const int umax = B * k;
  // up to 512 experts the one-row kernel takes every token count (one unit
  // per (token, slot) pair; 64-column down tiles for one token); beyond,
  // the B-row kernels
  const bool per_pair = E <= 512;
  // several tokens per pair: 512-row K-slices (16 rows per lane), so the
  // gate_up workgroups of four tokens fit in one round of the CUs, and
  // 256-column down tiles of 16 rows per lane
  const bool long_slices = per_pair && B > 1 && (gs_gu % (2 * kGuL)) == 0;
  const int t2 = long_slices ? host_ceil_div(H, 256) : per_pair ? dn_t2(1, H) : dn_t2(B, H);
  const int s1 = long_slices ? host_ceil_div(H, kGuRowLanes * 2 * kGuL) : fused_s1(H);
  uint64_t* mbox = reinterpret_cast<uint64_t*>(counters + kMailboxBase);
  // the gate_up part padded to a whole number of XCD rounds (blocks past
  // the real ones exit at once), so down workgroup i runs on XCD i % 8
  const int n_gu = (umax * fused_t1(MI) * s1 + 7) & ~7, n_dn = umax * t2;
  DecodePlan* gplan = ws ? (DecodePlan*)(ws + o_plan) : nullptr;
  uint16_t* act = ws ? (uint16_t*)(ws + o_act) : nullptr;
  float* prod = ws ? (float*)(ws + o_prod) : nullptr;
  // decode tiles for both projections, or neither
  const bool tiled = gu_t != nullptr && dn_t != nullptr;
  // the XCD-group kernel reads x and the logits in 16-byte pieces
  if (xcd_shape(B, H, MI) && (E % 8) == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)logits & 15) == 0 &&
      xcd_placement(stream)) {
    const int gr = gu_rows_per_lane(gs_gu);
    const int t1 = MI / kGuActCols, s1 = H / kNarrowRows, t2x = H / kTileCols;
    const int ng = B * k * t1, gslots = xcd_gslots(B, k, MI), gp = kXcd * gslots;
    // the shared expert's down projection in the launch (one token): computed by the combiners
    const int n_sd = sh_gu != nullptr ? 1 : 0;
    const int grid = gp * (s1 + t2x) + host_ceil_div(B * (H / kCombCols), kXcd) * kXcd;
    const int pairs = xcd_pair_rounds(B, k, MI);
    auto launch_x = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)x, (const uint16_t*)logits,
                         (const uint32_t*)gu_w, (const uint16_t*)gu_s, (const uint32_t*)dn_w, (const uint16_t*)dn_s,
                         (const uint32_t*)gu_t, (const uint32_t*)dn_t, (const uint16_t*)sh_gu,
                         (const uint16_t*)sh_dn, n_sd, B, E, k, H, MI, gs_gu, gs_dn, ng, gslots, pairs, gplan, mbox,
                         act, prod, counters,
                         (const uint16_t*)shared, (const uint16_t*)gate, (uint16_t*)out, (int64_t*)idx_out,
                         (uint16_t*)w_out);
    };
    if (E <= 512) {
      if (gr == 16) tiled ? launch_x(moe_decode_xcd_kernel<8, 16, true>) : launch_x(moe_decode_xcd_kernel<8, 16, false>);
      else tiled ? launch_x(moe_decode_xcd_kernel<8, 8, true>) : launch_x(moe_decode_xcd_kernel<8, 8, false>);
    } else {
      if (gr == 16) tiled ? launch_x(moe_decode_xcd_kernel<16, 16, true>) : launch_x(moe_decode_xcd_kernel<16, 16, false>);
      else tiled ? launch_x(moe_decode_xcd_kernel<16, 8, true>) : launch_x(moe_decode_xcd_kernel<16, 8, false>);
    }
    return (int)hipGetLastError();
  }
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(n_gu + n_dn), dim3(kThreads), 0, stream, (const uint16_t*)x,
                       (const uint16_t*)logits, (const uint32_t*)gu_w, (const uint16_t*)gu_s, (const uint32_t*)dn_w,
                       (const uint16_t*)dn_s, (const uint32_t*)(tiled ? gu_t : nullptr),
                       (const uint32_t*)(tiled ? dn_t : nullptr), B, E, k, H, MI, gs_gu, gs_dn, n_gu, gplan, mbox,
                       act, prod, counters,
                       (const uint16_t*)shared, (const uint16_t*)gate, (uint16_t*)out, (int64_t*)idx_out,
                       (uint16_t*)w_out);
  };
  if (long_slices) launch(moe_decode_fused_kernel<1, 2 * kGuL, 8, 16>);
  else if (B == 1 || per_pair) launch(moe_decode_fused_kernel<1>);
  else if (B == 2) launch(moe_decode_fused_kernel<2>);
  else launch(moe_decode_fused_kernel<4>);
  return (int)hipGetLastError();
}

int qmoe_moe_decode(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                    const void* dn_s, const void* shared, const void* gate, void* out, void* idx_out,
                    void* w_out, int B, int E, int k, int H, int MI, int gs_gu, int gs_dn, void* workspace,
                    size_t workspace_bytes, void* counters, void* stream) {
  if (decode_check(B, E, k, H, MI, gs_gu, gs_dn) != QMOE_OK || (shared == nullptr) != (gate == nullptr) ||
      qmoe_moe_decode_counters(B, k, H, MI) < 0 || counters == nullptr)
    return QMOE_EINVAL;
  if (workspace != nullptr && workspace_bytes < qmoe_moe_decode_workspace(B, k, H, MI)) return QMOE_EWORKSPACE;
  return decode_fused_launch(x, logits, gu_w, gu_s, dn_w, dn_s, nullptr, nullptr, shared, gate, out, idx_out, w_out,
                             B, E, k, H, MI, gs_gu, gs_dn, (char*)workspace, (int*)counters, (hipStream_t)stream);
}

int qmoe_moe_decode_tiled(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                          const void* dn_s, const void* gu_t, const void* dn_t, const void* shared, const void* gate,
                          void* out, void* idx_out, void* w_out, int B, int E, int k, int H, int MI, int gs_gu,
                          int gs_dn, void* workspace, size_t workspace_bytes, void* counters, void* stream) {
  if (decode_check(B, E, k, H, MI, gs_gu, gs_dn) != QMOE_OK || (shared == nullptr) != (gate == nullptr) ||
      (gu_t == nullptr) != (dn_t == nullptr) || ((uintptr_t)gu_t & 15) || ((uintptr_t)dn_t & 15) ||
      qmoe_moe_decode_counters(B, k, H, MI) < 0 || counters == nullptr)
    return QMOE_EINVAL;
  if (workspace != nullptr && workspace_bytes < qmoe_moe_decode_workspace(B, k, H, MI)) return QMOE_EWORKSPACE;
  return decode_fused_launch(x, logits, gu_w, gu_s, dn_w, dn_s, gu_t, dn_t, shared, gate, out, idx_out, w_out, B, E,
                             k, H, MI, gs_gu, gs_dn, (char*)workspace, (int*)counters, (hipStream_t)stream);
}

int qmoe_moe_block_decode(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                          const void* dn_s, const void* gu_t, const void* dn_t, const void* sh_gu, const void* sh_dn,
                          void* out, void* idx_out, void* w_out, int E, int k, int H, int MI, int gs_gu, int gs_dn,
                          void* counters, void* stream) {
  // one token on the XCD-group launch only (the caller runs the separate
  // shared-down GEMV and qmoe_moe_decode otherwise)
  if (decode_check(1, E, k, H, MI, gs_gu, gs_dn) != QMOE_OK || sh_gu == nullptr || sh_dn == nullptr ||
      (gu_t == nullptr) != (dn_t == nullptr) || ((uintptr_t)gu_t & 15) || ((uintptr_t)dn_t & 15) ||
      counters == nullptr || qmoe_moe_decode_counters(1, k, H, MI) < 0 ||
      !xcd_shape(1, H, MI) || (E % 8) != 0 || ((uintptr_t)x & 15) || ((uintptr_t)logits & 15) ||
      ((uintptr_t)sh_gu & 15) || ((uintptr_t)sh_dn & 15) || MI > 8 * 64 * 4 || !xcd_placement((hipStream_t)stream))
    return QMOE_EINVAL;
  return decode_fused_launch(x, logits, gu_w, gu_s, dn_w, dn_s, gu_t, dn_t, nullptr,
                             (const uint16_t*)sh_gu + 2 * MI, out, idx_out, w_out, 1, E, k, H, MI, gs_gu, gs_dn,
                             nullptr, (int*)counters, (hipStream_t)stream, sh_gu, sh_dn);
}

int qmoe_decode_tiles_gate_up(const void* gu_w, void* gu_t, int E, int H, int MI, int gs_gu, void* stream) {
  if (gu_w == nullptr || gu_t == nullptr || ((uintptr_t)gu_t & 15) || E < 1 || E > 65535 || H < kTileCols ||
      (H % kTileCols) ||
      MI < kGuActCols || (MI % kGuActCols) || gs_gu < 8 || (gs_gu % 8) || (H % gs_gu))
    return QMOE_EINVAL;
  const int t1 = MI / kGuActCols, s1 = H / kNarrowRows;
  hipLaunchKernelGGL(decode_tiles_kernel, dim3(s1 * t1, E), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint32_t*)gu_w, (uint32_t*)gu_t, H, 2 * MI / 8, 0, gu_rows_per_lane(gs_gu), MI, t1);
  return (int)hipGetLastError();
}

int qmoe_decode_tiles_down(const void* dn_w, void* dn_t, int E, int H, int MI, void* stream) {
  if (dn_w == nullptr || dn_t == nullptr || ((uintptr_t)dn_t & 15) || E < 1 || E > 65535 || H < kTileCols ||
      (H % kTileCols) ||
      MI < kGuActCols || (MI % kGuActCols))
    return QMOE_EINVAL;
  const int t1 = MI / kGuActCols, t2 = H / kTileCols;
  hipLaunchKernelGGL(decode_tiles_kernel, dim3(t1 * t2, E), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint32_t*)dn_w, (uint32_t*)dn_t, MI, H / 8, 1, kNarrowR, MI, t2);
  return (int)hipGetLastError();
}

int qmoe_xcd_placement(int mode, void* stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices || mode < 0 || mode > 2) return QMOE_EINVAL;
  if (mode != 0) {
    std::lock_guard<std::mutex> lock(g_place_mutex);
    g_place[dev] = mode == 1 ? kPlaceOther : kPlaceUnknown;
    return 0;
  }
  return xcd_placement((hipStream_t)stream) ? 1 : 0;
}

size_t qmoe_moe_decode_noalloc_max_bytes(void) { return kScratchBytes; }

int qmoe_moe_decode_noalloc(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                            const void* dn_s, const void* shared, const void* gate, void* out, void* idx_out,
                            void* w_out, int B, int E, int k, int H, int MI, int gs_gu, int gs_dn, void* stream) {
  if (decode_check(B, E, k, H, MI, gs_gu, gs_dn) != QMOE_OK || (shared == nullptr) != (gate == nullptr))
    return QMOE_EINVAL;
  const int need = qmoe_moe_decode_counters(B, k, H, MI);
  if (need < 0 || need > kScratchInts) return QMOE_ESCRATCH;
  hipStream_t st = (hipStream_t)stream;
  int rc = QMOE_OK;
  int* cnt = device_scratch(st, &rc);
  if (cnt == nullptr) return rc;
  return decode_fused_launch(x, logits, gu_w, gu_s, dn_w, dn_s, nullptr, nullptr, shared, gate, out, idx_out, w_out,
                             B, E, k, H, MI, gs_gu, gs_dn, nullptr, cnt, st);
}

int qmoe_moe_decode_status(const void* counters, int clear, int* flag_out, void* stream) {
  if (flag_out == nullptr) return QMOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  if (counters == nullptr) {
    int rc = QMOE_OK;
    counters = device_scratch(st, &rc);
    if (counters == nullptr) return rc;
  }
  int* flag = (int*)counters + kErrSlot;
  int host = 0;
  hipError_t e = hipMemcpyAsync(&host, flag, sizeof(int), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e == hipSuccess && clear && host) {
    const int zero = 0;
    e = hipMemcpyAsync(flag, &zero, sizeof(int), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
  }
  if (e != hipSuccess) return (int)e;
  *flag_out = host;
  return QMOE_OK;
}

}  // extern "C"
