// Router top-k and expert-major grouping on the GPU.
//
// Router: one wave per token; softmax over E logits, top-k by (logit desc,
// expert id asc), probabilities renormalised over the selection, bf16.
// (fnx/engine.py:1810-1813)
//
// Grouping (fnx/engine.py:1816-1823, 1832-1843), deterministic and stable:
//   1. count   : per chunk of 256 flat ids, an LDS histogram -> hist[c][e]
//   2. scan    : per expert, the chunk counts become each chunk's offset
//                within the expert's run (workgroups of 64 experts, the
//                chunks split over 4 thread groups) plus the expert total;
//                then one workgroup scans the totals into counts/ends (int64,
//                inclusive cumsum = group_list) and emits the grouped GEMM's
//                row-tile table (expert, first row, rows).
//   3. scatter : one wave per chunk (run bases = expert start + chunk offset)
//                walks its ids in flat order; an id's rank
//                among equal ids before it in the same wave step comes from
//                lane reads, so order[pos] = f is the stable expert-major order
//                and inverse[f] = pos.
// Ids outside [0, E) are not counted and not placed (inverse = -1).
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

constexpr int kChunk = 256;  // flat ids per chunk (one wave, 4 per lane)

template <int KPL>
__global__ __launch_bounds__(256) void router_topk_kernel(const uint16_t* __restrict__ logits,
                                                          int64_t* __restrict__ idx_out,
                                                          uint16_t* __restrict__ w_out, int T, int E, int k) {
  __shared__ int s_idx[4][QMOE_KMAX];
  __shared__ float s_w[4][QMOE_KMAX];
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // whole wave exits together
  wave_topk_softmax<KPL>(logits + (size_t)t * E, E, k, s_idx[wave], s_w[wave]);
  const int lane = threadIdx.x & 63;
  if (lane < k) {
    idx_out[(size_t)t * k + lane] = s_idx[wave][lane];
    w_out[(size_t)t * k + lane] = (uint16_t)f32_to_bf16(s_w[wave][lane]);
  }
}

__global__ __launch_bounds__(64) void route_count_kernel(const int64_t* __restrict__ ids, int R, int E,
                                                         int* __restrict__ hist) {
  extern __shared__ int lhist[];
  const int c = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += 64) lhist[e] = 0;
  __syncthreads();
  const int base = c * kChunk;
  // all of this lane's ids in flight at once
  int64_t v[kChunk / 64];
#pragma unroll
  for (int q = 0; q < kChunk / 64; ++q) {
    const int f = base + q * 64 + (int)threadIdx.x;
    v[q] = (f < R) ? ids[f] : -1;
  }
#pragma unroll
  for (int q = 0; q < kChunk / 64; ++q)
    if (v[q] >= 0 && v[q] < E) atomicAdd(&lhist[(int)v[q]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 64) hist[(size_t)c * E + e] = lhist[e];
}

// Per expert e (64 per workgroup): hist[c][e] <- sum_{c' < c} hist[c'][e]
// (offset of chunk c's run within the expert), tot[e] <- the total. Thread
// group g of 16 takes a contiguous sixteenth of the chunks; up to 16 chunks
// per thread are read in one batch and kept in registers for the rewrite
// (more chunks go in batches and are read again).
constexpr int kScanGroups = 16;
__global__ __launch_bounds__(1024) void route_chunk_scan_kernel(int* __restrict__ hist, int nchunks, int E,
                                                                 int* __restrict__ tot) {
  __shared__ int s_part[kScanGroups][64];
  const int el = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int e = blockIdx.x * 64 + el;
  const int per = (nchunks + kScanGroups - 1) / kScanGroups;
  const int c0 = min(nchunks, g * per), c1 = min(nchunks, c0 + per);
  int v[16];
  int sum = 0;
  if (e < E) {
    for (int c = c0; c < c1; c += 16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = (c + i < c1) ? hist[(size_t)(c + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) sum += v[i];
    }
  }
  s_part[g][el] = sum;
  __syncthreads();
  int b = 0;
  for (int q = 0; q < g; ++q) b += s_part[q][el];
  if (e < E) {
    if (g == kScanGroups - 1) tot[e] = b + sum;
    for (int c = c0; c < c1; c += 16) {
      if (c1 - c0 > 16) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = (c + i < c1) ? hist[(size_t)(c + i) * E + e] : 0;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (c + i < c1) {
          hist[(size_t)(c + i) * E + e] = b;
          b += v[i];
        }
    }
  }
}

// ---------------------------------------------------------------- row-tile table
//
// The grouped GEMM runs its row tiles in table order (every XCD takes every
// eighth tile, each with all its column tiles), so the table lists them
// longest first: every full tile (BM rows) in expert order, then each
// expert's partial last tile by rows descending, equal rows in expert order.
// The shortest tiles then fill the end of the launch instead of a long one
// running alone. Deterministic: ranks among equal row counts come from wave
// ballots and per-wave counts, not from atomics. BM above kLptMaxBM keeps
// expert order.
constexpr int kLptMaxBM = 256;
constexpr int kScanWaves = 16;  // 1024 threads

struct TileScratch {
  int w[kScanWaves];                 // per-wave sums of a block scan
  int h[kScanWaves][kLptMaxBM];      // per-wave counts of partial tiles by rows (one 1024-expert chunk)
  int cnt[kLptMaxBM];                // partial tiles by rows
  int run[kLptMaxBM];                // partial tiles by rows in earlier chunks
  int base[kLptMaxBM];               // first position of each row count among the partial tiles
};

// Exclusive prefix of v over the workgroup's threads in thread order; *total
// gets the sum. Every thread must call it.
QMOE_DEV int block_excl_scan(int v, int* s_w, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) s_w[wave] = incl;
  __syncthreads();
  int b = 0, t = 0;
  for (int q = 0; q < kScanWaves; ++q) {
    const int sq = s_w[q];
    if (q < wave) b += sq;
    t += sq;
  }
  __syncthreads();
  *total = t;
  return b + incl - v;
}

// Row tiles of E experts with s_tot[e] rows starting at row s_start[e] (LDS),
// at most max_tiles of them; tile_count = the number written.
QMOE_DEV void write_row_tiles(const int* s_tot, const int* s_start, int E, int BM, int max_tiles,
                              int* __restrict__ tile_expert, int* __restrict__ tile_row0,
                              int* __restrict__ tile_rows, int* __restrict__ tile_count, TileScratch& ts) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool lpt = BM <= kLptMaxBM;
  // rows / BM and rows % BM, with shifts when BM is a power of two
  const int sh = (BM & (BM - 1)) == 0 ? __builtin_ctz((unsigned)BM) : -1;
  auto tdiv = [&](int v) { return sh >= 0 ? v >> sh : v / BM; };
  auto tmod = [&](int v) { return sh >= 0 ? v & (BM - 1) : v % BM; };
  // full tiles (all tiles when not sorting), contiguous experts per thread
  const int per = (E + 1023) / 1024;
  const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
  auto full_of = [&](int e) { return lpt ? tdiv(s_tot[e]) : tdiv(s_tot[e] + BM - 1); };
  int mine = 0;
  for (int e = e0; e < e1; ++e) mine += full_of(e);
  int nfull = 0;
  int pos = block_excl_scan(mine, ts.w, &nfull);
  for (int e = e0; e < e1; ++e) {
    const int nf = full_of(e);
    for (int q = 0; q < nf; ++q, ++pos)
      if (pos < max_tiles) {
        tile_expert[pos] = e;
        tile_row0[pos] = s_start[e] + q * BM;
        tile_rows[pos] = min(BM, s_tot[e] - q * BM);
      }
  }
  if (!lpt) {
    if (tid == 0) tile_count[0] = min(nfull, max_tiles);
    return;
  }
  // Partial tiles. Per chunk of 1024 experts, thread t holds expert c0 + t
  // with r = rows % BM; wave ballots give its rank among the lanes of its wave
  // with the same r, and h[w][r] the count of such lanes in wave w.
  const int nchunks = (E + 1023) / 1024;
  int r = 0, rank_w = 0;
  auto chunk_ranks = [&](int c0) {
    for (int i = lane; i < BM; i += 64) ts.h[wave][i] = 0;  // this wave's row, written only by it
    const int e = c0 + tid;
    r = e < E ? tmod(s_tot[e]) : 0;
    uint64_t same = ~0ull;
    for (int bit = 0; bit < 8; ++bit) {
      const bool on = (r >> bit) & 1;
      const uint64_t bal = __ballot(on);
      same &= on ? bal : ~bal;
    }
    rank_w = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
    if (r && (lane == 63 || (same >> (lane + 1)) == 0ull)) ts.h[wave][r] = __popcll(same);
  };
  auto sum_h = [&](int i) {
    int v = 0;
#pragma unroll
    for (int q = 0; q < kScanWaves; ++q) v += ts.h[q][i];
    return v;
  };
  // pass 1: partial tiles by rows (cnt)
  for (int c = 0; c < nchunks; ++c) {
    chunk_ranks(c * 1024);
    __syncthreads();
    if (tid < BM) ts.cnt[tid] = (c ? ts.cnt[tid] : 0) + sum_h(tid);
    __syncthreads();
  }
  // base[r] = partial tiles with more rows than r: an exclusive scan over the
  // counts in descending row order (thread t holds row count BM - 1 - t)
  int npart = 0;
  {
    const int rr = BM - 1 - tid;
    const int before = block_excl_scan(rr > 0 ? ts.cnt[rr] : 0, ts.w, &npart);
    if (rr >= 0) ts.base[rr] = before;
    if (tid < BM) ts.run[tid] = 0;
  }
  __syncthreads();
  // pass 2: positions (one chunk: the ranks of pass 1 still hold)
  for (int c = 0; c < nchunks; ++c) {
    if (nchunks > 1) {
      chunk_ranks(c * 1024);
      __syncthreads();
    }
    if (r) {
      int rank = ts.run[r] + rank_w;
      for (int q = 0; q < wave; ++q) rank += ts.h[q][r];
      const int e = c * 1024 + tid;
      const int p = nfull + ts.base[r] + rank;
      if (p < max_tiles) {
        tile_expert[p] = e;
        tile_row0[p] = s_start[e] + (s_tot[e] - r);
        tile_rows[p] = r;
      }
    }
    if (nchunks > 1) {
      __syncthreads();
      if (tid < BM) ts.run[tid] += sum_h(tid);
      __syncthreads();
    }
  }
  if (tid == 0) tile_count[0] = min(nfull + npart, max_tiles);
}

// One workgroup of 1024 threads; E <= 4096: expert totals -> counts, ends
// and the row-tile table.
__global__ __launch_bounds__(1024) void route_scan_kernel(const int* __restrict__ tot_in, int E,
                                                          int64_t* __restrict__ counts, int64_t* __restrict__ ends,
                                                          int BM, int max_tiles, int* __restrict__ tile_expert,
                                                          int* __restrict__ tile_row0, int* __restrict__ tile_rows,
                                                          int* __restrict__ tile_count) {
  __shared__ int s_tot[4096];
  __shared__ int s_start[4096];
  __shared__ TileScratch ts;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) s_tot[e] = tot_in[e];
  __syncthreads();
  const int per = (E + 1023) / 1024;
  const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
  int run = 0;
  for (int e = e0; e < e1; ++e) run += s_tot[e];
  int total = 0;
  int start = block_excl_scan(run, ts.w, &total);
  for (int e = e0; e < e1; ++e) {
    const int tot = s_tot[e];
    counts[e] = tot;
    ends[e] = start + tot;
    s_start[e] = start;
    start += tot;
  }
  __syncthreads();
  if (tile_expert != nullptr)
    write_row_tiles(s_tot, s_start, E, BM, max_tiles, tile_expert, tile_row0, tile_rows, tile_count, ts);
}

__global__ __launch_bounds__(64) void route_scatter_kernel(const int64_t* __restrict__ ids, int R, int E,
                                                           const int* __restrict__ base,
                                                           const int64_t* __restrict__ counts,
                                                           const int64_t* __restrict__ ends,
                                                           int64_t* __restrict__ order,
                                                           int64_t* __restrict__ inverse) {
  extern __shared__ int run[];
  const int c = blockIdx.x;
  const int lane = threadIdx.x;
  const int nbits = 32 - __builtin_clz((unsigned)max(E - 1, 1));  // bits of an expert id
  // this lane's ids, then the run starts eight experts at a time, so the
  // global loads are in flight together rather than one round trip each
  int ev[kChunk / 64];
#pragma unroll
  for (int q = 0; q < kChunk / 64; ++q) {
    const int f = c * kChunk + q * 64 + lane;
    const int64_t v = (f < R) ? ids[f] : -1;
    ev[q] = (v >= 0 && v < E) ? (int)v : -1;
  }
  for (int e0 = lane; e0 < E; e0 += 8 * 64) {
    int r8[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + 64 * u;
      r8[u] = (e < E) ? (int)(ends[e] - counts[e]) + base[(size_t)c * E + e] : 0;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (e0 + 64 * u < E) run[e0 + 64 * u] = r8[u];
  }
  __syncthreads();
#pragma unroll
  for (int step = 0; step < kChunk / 64; ++step) {
    const int f = c * kChunk + step * 64 + lane;
    const int e = ev[step];
    // lanes holding the same id: intersect, bit by bit, the ballots of the
    // id's bits (invalid ids take the one key above every expert); then the
    // rank among lower lanes and whether this is the last one
    const int key = (e >= 0) ? e : (1 << nbits);
    uint64_t same = ~0ull;
    for (int b = 0; b <= nbits; ++b) {
      const bool bit = (key >> b) & 1;
      const uint64_t bal = __ballot(bit);
      same &= bit ? bal : ~bal;
    }
    const int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
    const bool last = (lane == 63) || ((same >> (lane + 1)) == 0ull);
    int pos = -1;
    if (e >= 0) pos = run[e] + rank;
    __syncthreads();  // every lane has read run[] before it is advanced
    if (e >= 0 && last) run[e] = pos + 1;
    if (f < R) {
      inverse[f] = pos;
      if (pos >= 0) order[pos] = f;
    }
    __syncthreads();
  }
}

// Row-tile table of the grouped GEMM from an inclusive cumulative group list
// (the grouped_matmul entry point, where rows are already expert-sorted).
__global__ __launch_bounds__(1024) void tiles_from_ends_kernel(const int64_t* __restrict__ ends, int E, int BM,
                                                               int R, int max_tiles, int* __restrict__ tile_expert,
                                                               int* __restrict__ tile_row0,
                                                               int* __restrict__ tile_rows,
                                                               int* __restrict__ tile_count) {
  __shared__ int s_tot[4096];
  __shared__ int s_start[4096];
  __shared__ TileScratch ts;
  for (int e = threadIdx.x; e < E; e += 1024) {
    const long b = e ? ends[e - 1] : 0, en = ends[e];
    const long bb = min(max(b, 0L), (long)R), ee = min(max(en, bb), (long)R);
    s_start[e] = (int)bb;
    s_tot[e] = (int)(ee - bb);
  }
  __syncthreads();
  write_row_tiles(s_tot, s_start, E, BM, max_tiles, tile_expert, tile_row0, tile_rows, tile_count, ts);
}

// Row-tile table with one tile per row: row j uses expert ids[j] (the
// decode down projection of row j with expert j, fnx/engine.py:703-721).
// Rows whose id lies outside [0, E) get an empty tile and stay unwritten.
__global__ __launch_bounds__(256) void tiles_from_ids_kernel(const int64_t* __restrict__ ids, int k, int E,
                                                             int* __restrict__ tile_expert, int* __restrict__ tile_row0,
                                                             int* __restrict__ tile_rows, int* __restrict__ tile_count) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j == 0) *tile_count = k;
  if (j >= k) return;
  const int64_t e = ids[j];
  const bool ok = e >= 0 && e < E;
  tile_expert[j] = ok ? (int)e : 0;
  tile_row0[j] = j;
  tile_rows[j] = ok ? 1 : 0;
}

}  // namespace

// ============================================================================ C ABI

extern "C" {

int qmoe_router_topk(const void* logits, void* idx_out, void* w_out, int T, int E, int k, void* stream) {
  if (T < 1 || E < 1 || E > 1024 || k < 1 || k > QMOE_KMAX || k > E) return QMOE_EINVAL;
  dim3 grid(host_ceil_div(T, 4));
  hipStream_t st = (hipStream_t)stream;
  if (E <= 512)
    hipLaunchKernelGGL((router_topk_kernel<8>), grid, dim3(256), 0, st, (const uint16_t*)logits,
                       (int64_t*)idx_out, (uint16_t*)w_out, T, E, k);
  else
    hipLaunchKernelGGL((router_topk_kernel<16>), grid, dim3(256), 0, st, (const uint16_t*)logits,
                       (int64_t*)idx_out, (uint16_t*)w_out, T, E, k);
  return (int)hipGetLastError();
}

// Workspace bytes for qmoe_route_group (chunk histograms, expert totals).
size_t qmoe_route_group_workspace(int R, int E) {
  return ((size_t)host_ceil_div(R, kChunk) + 1) * E * sizeof(int);
}

// Upper bound of grouped-GEMM row tiles for R rows over E experts.
int qmoe_max_row_tiles(int R, int E, int BM) { return host_ceil_div(R, BM) + E; }

int qmoe_route_group(const void* ids, int R, int E, void* counts, void* ends, void* order, void* inverse,
                     int BM, void* tile_expert, void* tile_row0, void* tile_rows, void* tile_count,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (R < 1 || E < 1 || E > 4096 || (tile_expert != nullptr && BM < 1)) return QMOE_EINVAL;
  if (workspace_bytes < qmoe_route_group_workspace(R, E)) return QMOE_EWORKSPACE;
  const int nchunks = host_ceil_div(R, kChunk);
  hipStream_t st = (hipStream_t)stream;
  int* hist = (int*)workspace;
  const size_t lds = (size_t)E * sizeof(int);
  hipLaunchKernelGGL(route_count_kernel, dim3(nchunks), dim3(64), lds, st, (const int64_t*)ids, R, E, hist);
  int* tot = hist + (size_t)nchunks * E;
  hipLaunchKernelGGL(route_chunk_scan_kernel, dim3(host_ceil_div(E, 64)), dim3(64 * kScanGroups), 0, st, hist, nchunks, E, tot);
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(1024), 0, st, (const int*)tot, E, (int64_t*)counts,
                     (int64_t*)ends, BM, qmoe_max_row_tiles(R, E, BM < 1 ? 1 : BM), (int*)tile_expert, (int*)tile_row0, (int*)tile_rows, (int*)tile_count);
  hipLaunchKernelGGL(route_scatter_kernel, dim3(nchunks), dim3(64), lds, st, (const int64_t*)ids, R, E,
                     (const int*)hist, (const int64_t*)counts, (const int64_t*)ends, (int64_t*)order,
                     (int64_t*)inverse);
  return (int)hipGetLastError();
}

int qmoe_tiles_from_ids(const void* ids, int k, int E, void* tile_expert, void* tile_row0, void* tile_rows,
                        void* tile_count, void* stream) {
  if (k < 1 || E < 1) return QMOE_EINVAL;
  hipLaunchKernelGGL(tiles_from_ids_kernel, dim3(host_ceil_div(k, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const int64_t*)ids, k, E, (int*)tile_expert, (int*)tile_row0, (int*)tile_rows, (int*)tile_count);
  return (int)hipGetLastError();
}

int qmoe_tiles_from_ends(const void* ends, int E, int R, int BM, void* tile_expert, void* tile_row0,
                         void* tile_rows, void* tile_count, void* stream) {
  if (E < 1 || E > 4096 || R < 0 || BM < 1) return QMOE_EINVAL;
  hipLaunchKernelGGL(tiles_from_ends_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const int64_t*)ends, E,
                     BM, R, qmoe_max_row_tiles(R, E, BM), (int*)tile_expert, (int*)tile_row0, (int*)tile_rows, (int*)tile_count);
  return (int)hipGetLastError();
}

}  // extern "C"
