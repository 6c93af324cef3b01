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
// pairs (W[k,n], W[k+1,n]) encoded as 1 + u/16 with u = q + 8 (nibble placed
// in the top mantissa bits, exponent 0), and dotted with (x[k], x[k+1]) by
// v_dot2c_f32_bf16 into an fp32 accumulator. Every product is exact in fp32;
// sum_k x*q = 16*acc - 24*sum_k x recovers the signed result. A thread's L
// rows lie in one scale group, so it applies S[g, n] once per run.
// Per-column results of the 32 row-lanes are summed in LDS in row-lane
// order, then across K-slices in slice order by the last workgroup to finish
// the tile (an atomic arrival counter that the finisher resets to zero), so
// results are deterministic run to run and no second launch is needed.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunks = 8;                     // 32-column chunks per tile
constexpr int kTileCols = kChunks * 32;        // 256
constexpr int kRowLanes = kThreads / kChunks;  // 32
constexpr int kRedStride = 36;                 // LDS floats per chunk (padded)
constexpr int kRedRow = kChunks * kRedStride;  // LDS floats per row-lane

// Byte-permute selectors for v_perm_b32(hi, lo, sel): bytes of the result,
// low to high, taken from {lo.b0..b3 = 0..3, hi.b0..b3 = 4..7}.
constexpr uint32_t kSelLo = 0x05040100u;  // lo.b0, lo.b1, hi.b0, hi.b1
constexpr uint32_t kSelHi = 0x07060302u;  // lo.b2, lo.b3, hi.b2, hi.b3

QMOE_DEV bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// Nibble j (0..3) of each 16-bit half of t -> bf16 pair 1 + u/16.
template <int J>
QMOE_DEV uint32_t nib_pair(uint32_t t) {
  uint32_t s = (J == 0) ? (t << 3) : (t >> (4 * J - 3));
  return (s & 0x00780078u) | 0x3f803f80u;
}

// One row pair (words a from row k, b from row k+1) of a 32-column chunk:
// acc[m][c] += x[m][k] * W'[k,c] + x[m][k+1] * W'[k+1,c] (W' = 1 + u/16).
template <int MR>
QMOE_DEV void dot_row_pair(const uint4& a, const uint4& b, const uint32_t* xp, float (*acc)[32]) {
  const uint32_t aw[4] = {a.x ^ 0x88888888u, a.y ^ 0x88888888u, a.z ^ 0x88888888u, a.w ^ 0x88888888u};
  const uint32_t bw[4] = {b.x ^ 0x88888888u, b.y ^ 0x88888888u, b.z ^ 0x88888888u, b.w ^ 0x88888888u};
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

template <int L>
QMOE_DEV void tile_load(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s, int N, int gs, int k0,
                        int kend, int colw, TileLoad<L>& t) {
  const int tid = threadIdx.x;
  const int r = tid / kChunks;
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

// Partial product of one workgroup from loaded weights: for m < MR and the
// tile's 256 columns,
//   out[m][col] = sum_{k in [k0, kend)} x[m][k] * q[k][col] * S[k/gs][col]
// written to red_out (LDS, [MR][256]) in column-tile order. AGENT_X reads x
// with device-coherent loads (x written by other workgroups of the launch).
template <int MR, int L, bool AGENT_X>
QMOE_DEV void tile_compute(const TileLoad<L>& t, const XRows& xr, int mrows, float* red, float* red_out) {
  const int tid = threadIdx.x;
  const int cc = tid & (kChunks - 1);
  const int r = tid / kChunks;

  float acc[MR][32];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[m][c] = 0.f;

  if (t.active) {
    uint32_t xp[MR][L / 2];
    float sx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      sx[m] = 0.f;
#pragma unroll
      for (int i = 0; i < L / 2; ++i) {
        uint32_t v = 0u;
        if (m < mrows) {
          const uint32_t* xa = reinterpret_cast<const uint32_t*>(xr.p[m] + t.kr + 2 * i);
          v = AGENT_X ? __hip_atomic_load(const_cast<uint32_t*>(xa), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *xa;
        }
        xp[m][i] = v;
        sx[m] += bf16_to_f32(v & 0xffffu) + bf16_to_f32(v >> 16);
      }
    }
#pragma unroll
    for (int i = 0; i < L / 2; ++i) {
      uint32_t xpi[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) xpi[m] = xp[m][i];
      dot_row_pair<MR>(t.wv[2 * i], t.wv[2 * i + 1], xpi, acc);
    }
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const float sc = bf16_to_f32((c & 1) ? (t.sw[c >> 1] >> 16) : (t.sw[c >> 1] & 0xffffu));
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m][c] = sc * (16.f * acc[m][c] - 24.f * sx[m]);
    }
  }

  // deterministic reduction over the 32 row-lanes, one row of x at a time
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float4* dst = reinterpret_cast<float4*>(red + r * kRedRow + cc * kRedStride);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      dst[q] = make_float4(acc[m][4 * q], acc[m][4 * q + 1], acc[m][4 * q + 2], acc[m][4 * q + 3]);
    __syncthreads();
    {
      const int col = tid;  // 0..255
      const float* src = red + (col >> 5) * kRedStride + (col & 31);
      float sum = 0.f;
#pragma unroll 8
      for (int rr = 0; rr < kRowLanes; ++rr) sum += src[rr * kRedRow];
      red_out[m * kTileCols + col] = sum;
    }
    __syncthreads();
  }
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

// ---------------------------------------------------------------- standalone GEMM (M <= 4)

template <int MR, int L>
__global__ __launch_bounds__(kThreads) void w4a16_gemv_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
    uint16_t* __restrict__ y, int M, int K, int N, int gs, float* __restrict__ part,
    int* __restrict__ counters) {
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[MR * kTileCols];
  const int ntile = blockIdx.x;
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
  w4_tile_partial<MR, L>(w, s, xr, M, K, N, gs, k0, kend, colw, red, res);

  const int col = ntile * kTileCols + threadIdx.x;
  float* mypart = part + ((size_t)slice * MR) * N;
  for (int m = 0; m < M; ++m)
    if (col < N) store_agent(&mypart[(size_t)m * N + col], res[m * kTileCols + threadIdx.x]);
  if (!arrive_last(counters + ntile, nslices)) return;
  if (col >= N) return;
  for (int m = 0; m < M; ++m) {
    const float sum = sum_agent_ordered(&part[(size_t)m * N + col], (size_t)MR * N, nslices);
    y[(size_t)m * N + col] = (uint16_t)f32_to_bf16(sum);
  }
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
};

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
    int u = 0;
    while (remaining != 0) {
      const int leader = __builtin_ctzll(remaining);
      const int el = __builtin_amdgcn_readlane(e, leader);
      const uint64_t match = __builtin_amdgcn_ballot_w64(valid && e == el);
      if ((match >> lane) & 1ull) {
        const int m = __builtin_popcountll(match & ((1ull << lane) - 1ull));
        if (m == 0) {
          plan.uexp[u] = e;
          plan.umult[u] = __builtin_popcountll(match);
        }
        plan.utok[u][m] = t;
        plan.uslot[u][m] = j;
      }
      remaining &= ~match;
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
// grid.x = (MI/128 column tiles) x (K-slices), grid.y = B*k unique slots.
template <int L>
__global__ __launch_bounds__(kThreads) void moe_decode_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ logits, const uint32_t* __restrict__ wgu,
    const uint16_t* __restrict__ sgu, int B, int E, int k, int H, int MI, int gs,
    DecodePlan* __restrict__ gplan, float* __restrict__ part, uint16_t* __restrict__ act,
    int* __restrict__ counters, int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out) {
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[kMaxTok * kTileCols];
  __shared__ DecodePlan plan;
  const int ntiles = (MI + 127) / 128;
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
  const int cc = threadIdx.x & (kChunks - 1);
  const int ic = tile * 128 + (cc & 3) * 32;  // intermediate column of the chunk
  const int col0 = (cc < 4) ? ic : MI + ic;
  const int colw = ic < MI ? (col0 >> 3) : -1;

  // rows of x of the tokens routed to this expert
  XRows xr;
#pragma unroll
  for (int m = 0; m < kMaxTok; ++m) xr.p[m] = x + (size_t)plan.utok[u][min(m, mult - 1)] * H;

  const uint32_t* we = wgu + (size_t)e * H * (N >> 3);
  const uint16_t* se = sgu + (size_t)e * (H / gs) * N;
  const int ks = kRowLanes * L;
  const int k0 = slice * ks;
  const int kend = min(H, k0 + ks);
  if (mult == 1) w4_tile_partial<1, L>(we, se, xr, 1, H, N, gs, k0, kend, colw, red, res);
  else if (mult == 2) w4_tile_partial<2, L>(we, se, xr, 2, H, N, gs, k0, kend, colw, red, res);
  else w4_tile_partial<4, L>(we, se, xr, mult, H, N, gs, k0, kend, colw, red, res);

  // partials: part[u][slice][m][tile][256]
  const size_t tile_stride = (size_t)ntiles * kTileCols;
  float* mypart = part + (((size_t)u * nslices + slice) * kMaxTok) * tile_stride + (size_t)tile * kTileCols;
  for (int m = 0; m < mult; ++m) store_agent(&mypart[(size_t)m * tile_stride + threadIdx.x], res[m * kTileCols + threadIdx.x]);
  if (!arrive_last(counters + u * ntiles + tile, nslices)) return;

  // last workgroup of this (expert, tile): reduce slices, SwiGLU, store act
  const int i = threadIdx.x & 127;
  const int half = threadIdx.x >> 7;
  const int col = tile * 128 + i;
  for (int m = half; m < mult; m += 2) {
    const float* p = part + ((size_t)u * nslices * kMaxTok + m) * tile_stride + (size_t)tile * kTileCols;
    const float g = sum_agent_ordered(p + i, kMaxTok * tile_stride, nslices);
    const float up = sum_agent_ordered(p + 128 + i, kMaxTok * tile_stride, nslices);
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
// grid.x = (H/256 column tiles) x (K-slices), grid.y = B*k unique slots.
template <int L>
__global__ __launch_bounds__(kThreads) void moe_decode_down_kernel(
    const uint32_t* __restrict__ wdn, const uint16_t* __restrict__ sdn, int B, int k, int H, int MI,
    int gs, const DecodePlan* __restrict__ gplan, const uint16_t* __restrict__ act,
    float* __restrict__ part, float* __restrict__ prod, int* __restrict__ counters,
    int* __restrict__ counters_out, const uint16_t* __restrict__ shared, const uint16_t* __restrict__ gate,
    uint16_t* __restrict__ out) {
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[kMaxTok * kTileCols];
  __shared__ DecodePlan plan;
  {
    const int* src = reinterpret_cast<const int*>(gplan);
    int* dst = reinterpret_cast<int*>(&plan);
    for (int q = threadIdx.x; q < (int)(sizeof(DecodePlan) / sizeof(int)); q += kThreads) dst[q] = src[q];
    __syncthreads();
  }
  const int ntiles = (H + kTileCols - 1) / kTileCols;
  const int tile = blockIdx.x % ntiles;
  const int slice = blockIdx.x / ntiles;
  const int nslices = gridDim.x / ntiles;
  const int u = blockIdx.y;
  const int nunique = plan.nunique;
  if (u >= nunique) return;
  const int e = plan.uexp[u];
  const int mult = plan.umult[u];
  const int cc = threadIdx.x & (kChunks - 1);
  const int col0 = tile * kTileCols + cc * 32;
  const int colw = col0 < H ? (col0 >> 3) : -1;
  const uint32_t* we = wdn + (size_t)e * MI * (H >> 3);
  const uint16_t* se = sdn + (size_t)e * (MI / gs) * H;
  XRows xr;
#pragma unroll
  for (int m = 0; m < kMaxTok; ++m) xr.p[m] = act + ((size_t)u * kMaxTok + min(m, mult - 1)) * MI;
  const int ks = kRowLanes * L;
  const int k0 = slice * ks;
  const int kend = min(MI, k0 + ks);
  if (mult == 1) w4_tile_partial<1, L>(we, se, xr, 1, MI, H, gs, k0, kend, colw, red, res);
  else if (mult == 2) w4_tile_partial<2, L>(we, se, xr, 2, MI, H, gs, k0, kend, colw, red, res);
  else w4_tile_partial<4, L>(we, se, xr, mult, MI, H, gs, k0, kend, colw, red, res);

  const size_t tile_stride = (size_t)ntiles * kTileCols;
  float* mypart = part + (((size_t)u * nslices + slice) * kMaxTok) * tile_stride + (size_t)tile * kTileCols;
  for (int m = 0; m < mult; ++m) store_agent(&mypart[(size_t)m * tile_stride + threadIdx.x], res[m * kTileCols + threadIdx.x]);
  if (!arrive_last(counters + u * ntiles + tile, nslices)) return;

  // expert output of this tile -> weighted bf16 products at (token, slot)
  const int col = tile * kTileCols + threadIdx.x;
  for (int m = 0; m < mult; ++m) {
    const float sum =
        sum_agent_ordered(&part[((size_t)u * nslices * kMaxTok + m) * tile_stride + col], kMaxTok * tile_stride, nslices);
    const int t = plan.utok[u][m], j = plan.uslot[u][m];
    if (col < H) store_agent(&prod[((size_t)t * k + j) * H + col], round_bf16(round_bf16(sum) * plan.w[t][j]));
  }
  if (!arrive_last(counters_out + tile, nunique)) return;

  // every expert of every token has contributed this tile: ordered combine
  if (col >= H) return;
  for (int t = 0; t < B; ++t) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) acc += load_agent(&prod[((size_t)t * k + j) * H + col]);
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
// One launch for the whole block, with two hand-offs between workgroups.
// Blocks [0, n_gu) are gate_up workgroups (unique slot u, 128-column tile,
// K-slice): they store their split-K partials of the gate and up columns and
// bump cnt_gu[u][tile]. Blocks [n_gu, grid) are down workgroups (u, 256-column
// tile, 128-row K-slice): they route, load their weights and scales (which
// depend only on the routing), then wait for the gate_up tile that holds
// their 128 act rows, sum its partials in slice order and apply SwiGLU
// themselves (so no workgroup has to publish act), and store their own
// partials. The last down block of each column tile sums every expert's
// partials in slice order and combines the top-k slots in slot order.
// Down blocks have higher indices than every gate_up block and workgroups of
// each XCD are dispatched in index order, so a waiting block never holds
// resources a block it waits for needs; the wait is also bounded and leaves
// an error flag instead of hanging. The last down block to pass its wait
// re-arms every cnt_gu for the next launch.
//
// Counter layout (int32): cnt_gu[umax*t1 * 32] (one per 128-byte line:
// hundreds of waiting blocks poll them) | cnt_rdy[1] | cnt_out[t2]; the error
// flag is the last slot of qmoe_moe_decode_counters().
constexpr int kSpinLimit = 1 << 22;  // polls (one agent-scope load each, about a microsecond)
constexpr int kFlagStride = 32;      // ints between polled counters (128 bytes)

template <int MRMAX>
__global__ __launch_bounds__(kThreads) void moe_decode_fused_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ logits, const uint32_t* __restrict__ wgu,
    const uint16_t* __restrict__ sgu, const uint32_t* __restrict__ wdn, const uint16_t* __restrict__ sdn, int B,
    int E, int k, int H, int MI, int gs_gu, int gs_dn, int n_gu, DecodePlan* __restrict__ gplan,
    float* __restrict__ part1, uint16_t* __restrict__ act, float* __restrict__ part2, float* __restrict__ prod,
    int* __restrict__ counters, int* __restrict__ err, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ out, int64_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out) {
  constexpr int L1 = 8, L2 = 4;
  static_assert(kRowLanes * L2 == 128, "a down K-slice is one gate_up column tile");
  __shared__ float red[kRowLanes * kRedRow];
  __shared__ float res[MRMAX * kTileCols];
  __shared__ DecodePlan plan;
  const int umax = B * k;
  const int t1 = (MI + 127) / 128, s1 = ceil_div(H, kRowLanes * L1);
  const int t2 = ceil_div(H, kTileCols), s2 = ceil_div(MI, kRowLanes * L2);
  int* cnt_gu = counters;
  int* cnt_rdy = cnt_gu + umax * t1 * kFlagStride;
  int* cnt_out = cnt_rdy + 1;

  const bool writer = blockIdx.x == 0;
  if (E <= 512) build_plan<8>(logits, B, E, k, plan, idx_out, w_out, writer);
  else build_plan<16>(logits, B, E, k, plan, idx_out, w_out, writer);
  if (writer) {
    const int* src = reinterpret_cast<const int*>(&plan);
    int* dst = reinterpret_cast<int*>(gplan);
    for (int q = threadIdx.x; q < (int)(sizeof(DecodePlan) / sizeof(int)); q += kThreads) dst[q] = src[q];
  }
  const int nunique = plan.nunique;
  const size_t stride1 = (size_t)t1 * kTileCols;  // part1[u][slice][m][tile][256]
  const size_t stride2 = (size_t)t2 * kTileCols;  // part2[u][slice][m][tile][256]

  if ((int)blockIdx.x < n_gu) {
    // ---- gate_up partials
    const int per_u = t1 * s1;
    const int u = blockIdx.x / per_u;
    const int tile = (blockIdx.x % per_u) % t1;
    const int slice = (blockIdx.x % per_u) / t1;
    if (u >= nunique) return;
    const int e = plan.uexp[u];
    const int mult = plan.umult[u];
    const int N = 2 * MI;
    const int cc = threadIdx.x & (kChunks - 1);
    const int ic = tile * 128 + (cc & 3) * 32;
    const int col0 = (cc < 4) ? ic : MI + ic;
    const int colw = ic < MI ? (col0 >> 3) : -1;
    XRows xr;
#pragma unroll
    for (int m = 0; m < kMaxTok; ++m) xr.p[m] = x + (size_t)plan.utok[u][min(m, mult - 1)] * H;
    const uint32_t* we = wgu + (size_t)e * H * (N >> 3);
    const uint16_t* se = sgu + (size_t)e * (H / gs_gu) * N;
    const int ks = kRowLanes * L1, k0 = slice * ks, kend = min(H, k0 + ks);
    TileLoad<L1> tl;
    tile_load<L1>(we, se, N, gs_gu, k0, kend, colw, tl);
    if (MRMAX == 1 || mult == 1) tile_compute<1, L1, false>(tl, xr, 1, red, res);
    else if (MRMAX == 2 || mult == 2) tile_compute<(MRMAX >= 2 ? 2 : 1), L1, false>(tl, xr, mult, red, res);
    else tile_compute<MRMAX, L1, false>(tl, xr, mult, red, res);
    float* mypart = part1 + (((size_t)u * s1 + slice) * kMaxTok) * stride1 + (size_t)tile * kTileCols;
    for (int m = 0; m < mult; ++m) store_agent(&mypart[(size_t)m * stride1 + threadIdx.x], res[m * kTileCols + threadIdx.x]);
    // partials complete, then they count towards cnt_gu[u][tile]
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(cnt_gu + (u * t1 + tile) * kFlagStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // ---- down partials
  const int bid = (int)blockIdx.x - n_gu;
  const int per_u = t2 * s2;
  const int u = bid / per_u;
  const int tile = (bid % per_u) % t2;
  const int slice = (bid % per_u) / t2;  // == the gate_up tile of its act rows
  if (u >= nunique) return;
  const int e = plan.uexp[u];
  const int mult = plan.umult[u];
  const int cc = threadIdx.x & (kChunks - 1);
  const int col0 = tile * kTileCols + cc * 32;
  const int colw = col0 < H ? (col0 >> 3) : -1;
  const uint32_t* we = wdn + (size_t)e * MI * (H >> 3);
  const uint16_t* se = sdn + (size_t)e * (MI / gs_dn) * H;
  const int k0 = slice * 128, kend = min(MI, k0 + 128);
  // the gate_up weights are on the critical path: let their loads go first
  // (these are needed only after the gate_up partials are in)
  __builtin_amdgcn_s_sleep(64);
  __builtin_amdgcn_s_sleep(64);
  TileLoad<L2> tl;
  tile_load<L2>(we, se, H, gs_dn, k0, kend, colw, tl);
  // wait until every gate_up slice of tile `slice` of u has stored its partials
  if (threadIdx.x == 0) {
    int polls = 0;
    while (__hip_atomic_load(cnt_gu + (u * t1 + slice) * kFlagStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < s1) {
      __builtin_amdgcn_s_sleep(2);
      if (++polls == kSpinLimit) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
  // count this block as past its wait; the last of all down blocks re-arms
  // every cnt_gu (all gate_up arrivals of the launch happened before any
  // wait ended). The result is only looked at when the block finishes.
  int prev_done = 0;
  if (threadIdx.x == 0) prev_done = __hip_atomic_fetch_add(cnt_rdy, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  auto finish = [&]() {
    if (threadIdx.x == 0 && prev_done == nunique * per_u - 1) {
      for (int q = 0; q < nunique * t1; ++q)
        __hip_atomic_store(cnt_gu + q * kFlagStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(cnt_rdy, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  // act rows k0..k0+127 of each token routed to u: gate/up sums over the
  // gate_up slices in slice order, then SwiGLU, into LDS (as bf16 pairs)
  __shared__ uint32_t s_act[kMaxTok][64];
  {
    float* sgu_sum = red;  // [mult][256] scratch
    for (int m = 0; m < mult; ++m) {
      const float* pp = part1 + ((size_t)u * s1 * kMaxTok + m) * stride1 + (size_t)slice * kTileCols + threadIdx.x;
      sgu_sum[m * kTileCols + threadIdx.x] = sum_agent_ordered(pp, kMaxTok * stride1, s1);
    }
    __syncthreads();
    for (int q = threadIdx.x; q < mult * 64; q += kThreads) {
      const int m = q >> 6, i = 2 * (q & 63);
      const float* gsum = sgu_sum + m * kTileCols;
      const uint32_t a0 = f32_to_bf16(silu_f32(round_bf16(gsum[i])) * round_bf16(gsum[128 + i]));
      const uint32_t a1 = f32_to_bf16(silu_f32(round_bf16(gsum[i + 1])) * round_bf16(gsum[128 + i + 1]));
      s_act[m][q & 63] = a0 | (a1 << 16);
      // one copy of act for inspection (tile 0's blocks)
      if (tile == 0 && k0 + i < MI)
        *reinterpret_cast<uint32_t*>(act + ((size_t)u * kMaxTok + m) * MI + k0 + i) = a0 | (a1 << 16);
    }
    __syncthreads();
  }
  XRows xr;
#pragma unroll
  for (int m = 0; m < kMaxTok; ++m)
    xr.p[m] = reinterpret_cast<const uint16_t*>(&s_act[min(m, mult - 1)][0]) - k0;
  if (MRMAX == 1 || mult == 1) tile_compute<1, L2, false>(tl, xr, 1, red, res);
  else if (MRMAX == 2 || mult == 2) tile_compute<(MRMAX >= 2 ? 2 : 1), L2, false>(tl, xr, mult, red, res);
  else tile_compute<MRMAX, L2, false>(tl, xr, mult, red, res);
  float* mypart = part2 + (((size_t)u * s2 + slice) * kMaxTok) * stride2 + (size_t)tile * kTileCols;
  for (int m = 0; m < mult; ++m) store_agent(&mypart[(size_t)m * stride2 + threadIdx.x], res[m * kTileCols + threadIdx.x]);
  if (!arrive_last(cnt_out + tile, nunique * s2)) {
    finish();
    return;
  }
  finish();
  // last down block of this column tile: per token, the top-k slots in slot
  // order; each slot's expert output is its partials summed in slice order
  __shared__ int s_um[kMaxTok][QMOE_KMAX];
  if (threadIdx.x < umax) {
    // inverse of the plan: (token, slot) -> (unique slot, row)
    const int uu = threadIdx.x;
    if (uu < nunique)
      for (int m = 0; m < plan.umult[uu]; ++m) s_um[plan.utok[uu][m]][plan.uslot[uu][m]] = uu * kMaxTok + m;
  }
  __syncthreads();
  const int col = tile * kTileCols + threadIdx.x;
  if (col >= H) return;
  for (int t = 0; t < B; ++t) {
    float accv = 0.f;
    // all k (<= 16) slots at once, their partial loads (up to four slices
    // each per round) in flight together
    for (int j0 = 0; j0 < k; j0 += QMOE_KMAX) {
      float y[QMOE_KMAX];
#pragma unroll
      for (int jj = 0; jj < QMOE_KMAX; ++jj) y[jj] = 0.f;
      for (int b = 0; b < s2; b += 4) {
        float v[QMOE_KMAX][4];
#pragma unroll
        for (int jj = 0; jj < QMOE_KMAX; ++jj) {
          const int um = s_um[t][min(j0 + jj, k - 1)], uu = um / kMaxTok, m = um % kMaxTok;
          const float* pp = part2 + ((size_t)uu * s2 * kMaxTok + m) * stride2 + col;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[jj][i] = load_agent(pp + (size_t)min(b + i, s2 - 1) * kMaxTok * stride2);
        }
#pragma unroll
        for (int jj = 0; jj < QMOE_KMAX; ++jj)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (b + i < s2) y[jj] += v[jj][i];
      }
#pragma unroll
      for (int jj = 0; jj < QMOE_KMAX; ++jj) {
        const int j = j0 + jj;
        if (j < k) {
          const float pr = round_bf16(round_bf16(y[jj]) * plan.w[t][j]);
          prod[((size_t)t * k + j) * H + col] = pr;  // for inspection
          accv += pr;
        }
      }
    }
    float r = round_bf16(accv);
    if (shared != nullptr) {
      const float g = bf16_to_f32(gate[t]);
      const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
      r = round_bf16(r + round_bf16(bf16_to_f32(shared[(size_t)t * H + col]) * sg));
    }
    out[(size_t)t * H + col] = (uint16_t)f32_to_bf16(r);
  }
}

}  // namespace

// ============================================================================ C ABI

extern "C" {

// Workspace bytes needed by qmoe_w4a16_gemm for an [M,K]x[K,N] call.
size_t qmoe_w4a16_gemm_workspace(int M, int K, int N) {
  (void)M;
  const int nslices = host_ceil_div(K, kRowLanes * 4);
  return (size_t)nslices * 4 * (size_t)N * sizeof(float);
}

// Counter slots needed by qmoe_w4a16_gemm (int32, zero on first use).
int qmoe_w4a16_gemm_counters(int N) { return host_ceil_div(N, kTileCols); }

int qmoe_w4a16_gemv(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                    int group_size, void* workspace, size_t workspace_bytes, void* counters,
                    void* stream) {
  if (M < 1 || M > 4 || K < 8 || N < 32 || (N % 32) || (K % 8) || group_size < 8 ||
      (group_size % 8) || (K % group_size))
    return QMOE_EINVAL;
  constexpr int L = 4;
  const int nslices = host_ceil_div(K, kRowLanes * L);
  if (workspace_bytes < qmoe_w4a16_gemm_workspace(M, K, N)) return QMOE_EWORKSPACE;
  dim3 grid(host_ceil_div(N, kTileCols), nslices);
  hipStream_t st = (hipStream_t)stream;
  auto* xp = (const uint16_t*)x;
  auto* wp = (const uint32_t*)w;
  auto* sp = (const uint16_t*)scale;
  auto* yp = (uint16_t*)y;
  auto* part = (float*)workspace;
  auto* cnt = (int*)counters;
  if (M == 1) hipLaunchKernelGGL((w4a16_gemv_kernel<1, L>), grid, dim3(kThreads), 0, st, xp, wp, sp, yp, M, K, N, group_size, part, cnt);
  else if (M == 2) hipLaunchKernelGGL((w4a16_gemv_kernel<2, L>), grid, dim3(kThreads), 0, st, xp, wp, sp, yp, M, K, N, group_size, part, cnt);
  else hipLaunchKernelGGL((w4a16_gemv_kernel<4, L>), grid, dim3(kThreads), 0, st, xp, wp, sp, yp, M, K, N, group_size, part, cnt);
  return (int)hipGetLastError();
}

// Workspace layout of qmoe_moe_decode (byte offsets), shared with the host.
static void decode_layout(int B, int k, int H, int MI, size_t* off_plan, size_t* off_part1,
                          size_t* off_act, size_t* off_part2, size_t* off_prod, size_t* total,
                          int* s1, int* s2) {
  constexpr int L1 = 8, L2 = 4;
  const int umax = B * k;
  const int t1 = (MI + 127) / 128, t2 = host_ceil_div(H, kTileCols);
  *s1 = host_ceil_div(H, kRowLanes * L1);
  *s2 = host_ceil_div(MI, kRowLanes * L2);
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o += (bytes + 255) & ~(size_t)255; return at; };
  *off_plan = take(sizeof(DecodePlan));
  *off_part1 = take((size_t)umax * (*s1) * kMaxTok * t1 * kTileCols * sizeof(float));
  *off_act = take((size_t)umax * kMaxTok * MI * sizeof(uint16_t));
  *off_part2 = take((size_t)umax * (*s2) * kMaxTok * t2 * kTileCols * sizeof(float));
  *off_prod = take((size_t)B * k * H * sizeof(float));
  *total = o;
}

size_t qmoe_moe_decode_workspace(int B, int k, int H, int MI) {
  size_t a, b, c, d, e, total;
  int s1, s2;
  decode_layout(B, k, H, MI, &a, &b, &c, &d, &e, &total, &s1, &s2);
  return total;
}

int qmoe_moe_decode_layout(int B, int k, int H, int MI, size_t* off_plan, size_t* off_act, size_t* off_prod) {
  if (B < 1 || B > kMaxTok || k < 1 || k > QMOE_KMAX || H < 1 || MI < 1) return QMOE_EINVAL;
  size_t part1, part2, total;
  int s1, s2;
  decode_layout(B, k, H, MI, off_plan, &part1, off_act, &part2, off_prod, &total, &s1, &s2);
  return QMOE_OK;
}

int qmoe_moe_decode_counters(int B, int k, int H, int MI) {
  const int umax = B * k;
  const int t1 = (MI + 127) / 128, t2 = host_ceil_div(H, kTileCols);
  // fused launch: cnt_gu (one per 128-byte line) | cnt_rdy | cnt_out; the
  // two separate launches: cnt_gu | cnt_dn | cnt_out; then the error flag
  const int fused = umax * t1 * 32 + 1 + t2;
  const int separate = umax * t1 + umax * t2 + t2;
  return std::max(fused, separate) + 1;
}

static int decode_check(int B, int E, int k, int H, int MI, int gs_gu, int gs_dn) {
  if (B < 1 || B > kMaxTok || k < 1 || k > QMOE_KMAX || E < k || E > 1024 || H < 32 || (H % 32) ||
      H > 8192 || MI < 32 || (MI % 32) || gs_gu < 8 || (gs_gu % 8) || (H % gs_gu) || gs_dn < 8 ||
      (gs_dn % 8) || (MI % gs_dn))
    return QMOE_EINVAL;
  return QMOE_OK;
}

int qmoe_moe_decode_gate_up(const void* x, const void* logits, const void* gu_w, const void* gu_s, void* idx_out,
                            void* w_out, int B, int E, int k, int H, int MI, int gs_gu, void* workspace,
                            size_t workspace_bytes, void* counters, void* stream) {
  if (decode_check(B, E, k, H, MI, gs_gu, 32) != QMOE_OK) return QMOE_EINVAL;
  size_t o_plan, o_part1, o_act, o_part2, o_prod, total;
  int s1, s2;
  decode_layout(B, k, H, MI, &o_plan, &o_part1, &o_act, &o_part2, &o_prod, &total, &s1, &s2);
  if (workspace_bytes < total) return QMOE_EWORKSPACE;
  char* ws = (char*)workspace;
  const int umax = B * k;
  const int t1 = (MI + 127) / 128;
  hipLaunchKernelGGL((moe_decode_gate_up_kernel<8>), dim3(t1 * s1, umax), dim3(kThreads), 0, (hipStream_t)stream,
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
  size_t o_plan, o_part1, o_act, o_part2, o_prod, total;
  int s1, s2;
  decode_layout(B, k, H, MI, &o_plan, &o_part1, &o_act, &o_part2, &o_prod, &total, &s1, &s2);
  if (workspace_bytes < total) return QMOE_EWORKSPACE;
  char* ws = (char*)workspace;
  const int umax = B * k;
  const int t1 = (MI + 127) / 128, t2 = host_ceil_div(H, kTileCols);
  int* cnt2 = (int*)counters + umax * t1;
  int* cnt3 = cnt2 + umax * t2;
  hipLaunchKernelGGL((moe_decode_down_kernel<4>), dim3(t2 * s2, umax), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint32_t*)dn_w, (const uint16_t*)dn_s, B, k, H, MI, gs_dn,
                     (const DecodePlan*)(ws + o_plan), (const uint16_t*)(ws + o_act), (float*)(ws + o_part2),
                     (float*)(ws + o_prod), cnt2, cnt3, (const uint16_t*)shared, (const uint16_t*)gate,
                     (uint16_t*)out);
  return (int)hipGetLastError();
}

int qmoe_moe_decode(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                    const void* dn_s, const void* shared, const void* gate, void* out, void* idx_out,
                    void* w_out, int B, int E, int k, int H, int MI, int gs_gu, int gs_dn, void* workspace,
                    size_t workspace_bytes, void* counters, void* stream) {
  if (decode_check(B, E, k, H, MI, gs_gu, gs_dn) != QMOE_OK || (shared == nullptr) != (gate == nullptr))
    return QMOE_EINVAL;
  size_t o_plan, o_part1, o_act, o_part2, o_prod, total;
  int s1, s2;
  decode_layout(B, k, H, MI, &o_plan, &o_part1, &o_act, &o_part2, &o_prod, &total, &s1, &s2);
  if (workspace_bytes < total) return QMOE_EWORKSPACE;
  char* ws = (char*)workspace;
  const int umax = B * k;
  const int t1 = (MI + 127) / 128, t2 = host_ceil_div(H, kTileCols);
  const int n_gu = umax * t1 * s1, n_dn = umax * t2 * s2;
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(n_gu + n_dn), dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                       (const uint16_t*)logits, (const uint32_t*)gu_w, (const uint16_t*)gu_s, (const uint32_t*)dn_w,
                       (const uint16_t*)dn_s, B, E, k, H, MI, gs_gu, gs_dn, n_gu, (DecodePlan*)(ws + o_plan),
                       (float*)(ws + o_part1), (uint16_t*)(ws + o_act), (float*)(ws + o_part2), (float*)(ws + o_prod),
                       (int*)counters, (int*)counters + qmoe_moe_decode_counters(B, k, H, MI) - 1,
                       (const uint16_t*)shared, (const uint16_t*)gate, (uint16_t*)out, (int64_t*)idx_out,
                       (uint16_t*)w_out);
  };
  if (B == 1) launch(moe_decode_fused_kernel<1>);
  else if (B == 2) launch(moe_decode_fused_kernel<2>);
  else launch(moe_decode_fused_kernel<4>);
  return (int)hipGetLastError();
}

}  // extern "C"
