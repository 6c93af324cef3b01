// Expert-major grouped W4A16 GEMM on bf16 MFMA (gfx950), for prefill.
//
//   y[p, n] = bf16( sum_g S[e_p, g, n] * sum_{k in group g} a[p, k] * q[e_p, k, n] )
//
// Rows p are sorted by expert; a row-tile table (expert, first row, rows)
// produced on the GPU by the routing scan drives the grid, so empty experts
// cost nothing and no host synchronisation is needed.
//
// Tile: 128 rows x 128 columns per workgroup (4 waves, each 64 x 64 = 4 x 4
// MFMA 16x16x32 tiles), K step 32. Per step the workgroup stages
//   A: 128 x 32 bf16 (rows gathered through an optional permutation), and
//   B: 32 x 128 int4 -> exact signed bf16 (q in -8..7 is exact in bf16),
// into a double-buffered LDS tile, B stored column-major so each lane's MFMA
// operand (8 consecutive k of one column) is one 16-byte LDS read. Products
// x*q are exact; each scale group accumulates in its own fp32 registers and
// is folded into the output accumulator as acc += S[g, n] * acc_g, so the
// weights are never rounded to bf16 (the scale stays exact in fp32).
//
// Epilogues: 0 = store bf16 rows; 1 = SwiGLU (the tile's columns are
// act columns [n0, n0+64) of the gate half and the same columns of the up
// half, paired in the same lane); 2 = down projection with the top-k weight
// folded in: prod[order[p], n] = bf16(bf16(y) * w[order[p]]), scattered to
// token-major rows for the ordered slot reduction.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDS_A = BK + 8;  // bf16 per staged A row (16-byte padding)
constexpr int LDS_B = BK + 8;  // bf16 per staged B column
constexpr int kThreads = 256;

struct GemmArgs {
  const uint16_t* a;         // activations, row stride lda (bf16)
  int lda;
  const int64_t* perm;       // mode 1: a row = a[perm[p] / topk]; mode 2: out row = perm[p]
  int topk;
  const uint32_t* w;         // int4pack [E, K, N/8]
  const uint16_t* s;         // bf16 scales [E, G, N]
  int K, N, gs;
  const int* tile_expert;    // row-tile table (nullptr: dense, one expert, R rows)
  const int* tile_row0;
  const int* tile_rows;
  const int* tile_count;
  int R;
  int n_ntiles;
  uint16_t* y;               // output
  int ldy;
  int MI;                    // mode 1: act width (gate half = [0, MI), up half = [MI, 2MI))
  const uint16_t* wts;       // mode 2: bf16 routing weights, flat [T*topk]
};

QMOE_DEV uint32_t pack_bf16_pair_exact(float lo, float hi) {
  // both values are small integers, exact in bf16: keep the high halves
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void grouped_gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_A];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_B];

  const int nblk = gridDim.x;
  const int logical = xcd_remap(blockIdx.x, nblk);
  const int mt = logical / g.n_ntiles;
  const int nt = logical % g.n_ntiles;
  int e, row0, rows;
  if (g.tile_expert != nullptr) {
    if (mt >= g.tile_count[0]) return;
    e = g.tile_expert[mt];
    row0 = g.tile_row0[mt];
    rows = g.tile_rows[mt];
  } else {
    e = 0;
    row0 = mt * BM;
    if (row0 >= g.R) return;
    rows = min(BM, g.R - row0);
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int N = g.N, K = g.K;
  const int nw = N >> 3;

  // global column of B-tile local column c
  const int n0 = (MODE == 1) ? nt * 64 : nt * BN;
  auto gcol = [&](int c) -> int {
    if (MODE == 1) return (c < 64) ? n0 + c : g.MI + n0 + c - 64;
    return n0 + c;
  };
  auto col_ok = [&](int c) -> bool {
    if (MODE == 1) return n0 + (c & 63) < g.MI;
    return n0 + c < N;
  };

  const uint32_t* we = g.w + (size_t)e * K * nw;
  const uint16_t* se = g.s + (size_t)e * (K / g.gs) * N;

  // ---- global -> register staging assignments
  // A: chunks tid and tid+256 of 512 (row = chunk/4, 8 k per chunk)
  const uint16_t* arow[2];
  bool aok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int ch = tid + h * kThreads;
    const int r = ch >> 2;
    aok[h] = r < rows;
    int src = row0 + min(r, rows - 1);
    if (MODE == 1 && g.perm != nullptr) src = (int)(g.perm[src] / g.topk);
    arow[h] = g.a + (size_t)src * g.lda + (ch & 3) * 8;
  }
  // B: row pair rp (rows 2rp, 2rp+1 of the step), 8 columns cg*8..cg*8+7
  const int rp = tid >> 4, cg = tid & 15;
  const bool bok = col_ok(cg * 8);
  const int bword = gcol(cg * 8) >> 3;

  uint4 areg[2];
  uint32_t breg[2];
  auto load_step = [&](int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      areg[h] = aok[h] ? *reinterpret_cast<const uint4*>(arow[h] + k0) : make_uint4(0, 0, 0, 0);
    if (bok) {
      breg[0] = we[(size_t)(k0 + 2 * rp) * nw + bword];
      breg[1] = we[(size_t)(k0 + 2 * rp + 1) * nw + bword];
    } else {
      breg[0] = breg[1] = 0u;
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = tid + h * kThreads;
      *reinterpret_cast<uint4*>(&As[buf][(ch >> 2) * LDS_A + (ch & 3) * 8]) = areg[h];
    }
    const int a = (int)breg[0], b = (int)breg[1];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float lo = (float)(int)__builtin_amdgcn_sbfe(a, 4 * j, 4);
      const float hi = (float)(int)__builtin_amdgcn_sbfe(b, 4 * j, 4);
      *reinterpret_cast<uint32_t*>(&Bs[buf][(cg * 8 + j) * LDS_B + 2 * rp]) = pack_bf16_pair_exact(lo, hi);
    }
  };

  // ---- accumulators
  f32x4_t acc[4][4], accg[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      accg[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  // wave's B-tile local column base of MFMA column tile tn
  int cb[4];
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) cb[tn] = (tn < 2) ? 32 * wn + 16 * tn : 64 + 32 * wn + 16 * (tn - 2);
  int rt_live = 0;  // MFMA row tiles of this wave holding real rows
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) rt_live += (64 * wm + 16 * tm < rows) ? 1 : 0;

  const int nsteps = K / BK;
  const int steps_per_group = g.gs / BK;
  load_step(0);
  store_step(0);
  __syncthreads();

  for (int ks = 0; ks < nsteps; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nsteps) load_step((ks + 1) * BK);
    if (rt_live > 0) {
      bf16x8_t bf[4];
#pragma unroll
      for (int tn = 0; tn < 4; ++tn)
        bf[tn] = *reinterpret_cast<const bf16x8_t*>(&Bs[cur][(cb[tn] + (lane & 15)) * LDS_B + 8 * (lane >> 4)]);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        if (tm < rt_live) {
          const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
              &As[cur][(64 * wm + 16 * tm + (lane & 15)) * LDS_A + 8 * (lane >> 4)]);
#pragma unroll
          for (int tn = 0; tn < 4; ++tn)
            accg[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[tn], accg[tm][tn], 0, 0, 0);
        }
      }
    }
    if (ks + 1 < nsteps) store_step(cur ^ 1);
    // fold a finished scale group into the output accumulators
    if ((ks + 1) % steps_per_group == 0) {
      const int grp = ks / steps_per_group;
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        const int c = cb[tn] + (lane & 15);
        const float sc = col_ok(c) ? bf16_to_f32(se[(size_t)grp * N + gcol(c)]) : 0.f;
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[tm][tn][i] += sc * accg[tm][tn][i];
            accg[tm][tn][i] = 0.f;
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue. MFMA 16x16 output layout: lane holds column lane%16 of
  // rows 4*(lane/16) + i, i = 0..3.
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 64 * wm + 16 * tm + 4 * (lane >> 4) + i;
      if (r >= rows) continue;
      const int p = row0 + r;
      if (MODE == 1) {
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
          const int c = cb[tn] + (lane & 15);  // gate-half local column (< 64)
          if (!col_ok(c)) continue;
          const float gv = round_bf16(acc[tm][tn][i]);
          const float uv = round_bf16(acc[tm][tn + 2][i]);
          g.y[(size_t)p * g.ldy + n0 + c] = (uint16_t)f32_to_bf16(silu_f32(gv) * uv);
        }
      } else if (MODE == 2) {
        const int64_t f = g.perm[p];
        const float wv = bf16_to_f32(g.wts[f]);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          const int c = cb[tn] + (lane & 15);
          if (!col_ok(c)) continue;
          g.y[(size_t)f * g.ldy + gcol(c)] = (uint16_t)f32_to_bf16(round_bf16(acc[tm][tn][i]) * wv);
        }
      } else {
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          const int c = cb[tn] + (lane & 15);
          if (!col_ok(c)) continue;
          g.y[(size_t)p * g.ldy + gcol(c)] = (uint16_t)f32_to_bf16(acc[tm][tn][i]);
        }
      }
    }
  }
}

// out[t, n] = bf16(sum_{j < k, in order} prod[t*k + j, n]) (+ shared, a bf16 add)
__global__ __launch_bounds__(256) void slot_reduce_kernel(const uint16_t* __restrict__ prod, int T, int k, int H,
                                                          const uint16_t* __restrict__ shared,
                                                          uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int c2 = blockIdx.x * 256 + threadIdx.x;  // pair of columns
  if (2 * c2 >= H) return;
  float a0 = 0.f, a1 = 0.f;
  for (int j = 0; j < k; ++j) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(prod + ((size_t)t * k + j) * H + 2 * c2);
    a0 += bf16_to_f32(v & 0xffffu);
    a1 += bf16_to_f32(v >> 16);
  }
  uint32_t r0 = f32_to_bf16(a0), r1 = f32_to_bf16(a1);
  if (shared != nullptr) {
    const uint32_t sv = *reinterpret_cast<const uint32_t*>(shared + (size_t)t * H + 2 * c2);
    r0 = f32_to_bf16(bf16_to_f32(r0) + bf16_to_f32(sv & 0xffffu));
    r1 = f32_to_bf16(bf16_to_f32(r1) + bf16_to_f32(sv >> 16));
  }
  *reinterpret_cast<uint32_t*>(out + (size_t)t * H + 2 * c2) = r0 | (r1 << 16);
}

template <int MODE>
int launch_gemm(const GemmArgs& a, int mtiles_max, hipStream_t st) {
  const int nblk = mtiles_max * a.n_ntiles;
  if (nblk <= 0) return 0;
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE>), dim3(nblk), dim3(kThreads), 0, st, a);
  return (int)hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// ============================================================================ C ABI

extern "C" {

int qmoe_gemm_tile_rows(void) { return BM; }

// Grouped GEMM over expert-sorted rows (npu_grouped_matmul, split_item 3,
// group_type 0). The row-tile table comes from qmoe_route_group or
// qmoe_tiles_from_ends; mtiles_max bounds the grid (qmoe_max_row_tiles).
int qmoe_grouped_gemm(const void* x, int R, int K, int N, int E, int gs, const void* w, const void* scale,
                      const void* tile_expert, const void* tile_row0, const void* tile_rows,
                      const void* tile_count, int mtiles_max, void* y, void* stream) {
  if (R < 0 || K < BK || (K % BK) || N < 8 || (N % 8) || E < 1 || gs < BK || (gs % BK) || (K % gs) ||
      !aligned16(x) || tile_expert == nullptr)
    return QMOE_EINVAL;
  if (R == 0) return 0;
  GemmArgs a{};
  a.a = (const uint16_t*)x; a.lda = K; a.perm = nullptr; a.topk = 1;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(N, BN); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, mtiles_max, (hipStream_t)stream);
}

// Dense W4A16 GEMM for M > 4 rows (one weight matrix, no routing).
int qmoe_w4a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int gs,
                         void* stream) {
  if (M < 1 || K < BK || (K % BK) || N < 8 || (N % 8) || gs < BK || (gs % BK) || (K % gs) || !aligned16(x))
    return QMOE_EINVAL;
  GemmArgs a{};
  a.a = (const uint16_t*)x; a.lda = K; a.topk = 1;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.R = M; a.n_ntiles = host_ceil_div(N, BN); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, host_ceil_div(M, BM), (hipStream_t)stream);
}

// Fused prefill expert path after routing: gate_up grouped GEMM on rows
// gathered through order (x row = order[p] / topk) with the SwiGLU epilogue,
// then the down grouped GEMM with the routing weight folded into its
// epilogue and scattered to token-major rows, then the ordered slot
// reduction (+ optional shared-expert output).
//   workspace: act [R, MI] bf16 then prod [R, H] bf16
size_t qmoe_moe_prefill_workspace(int T, int k, int H, int MI) {
  const size_t R = (size_t)T * k;
  return ((R * MI * 2 + 255) & ~(size_t)255) + R * H * 2;
}

int qmoe_moe_experts_grouped(const void* x, int T, int H, int MI, int E, int k, const void* wts,
                             const void* order, const void* gu_w, const void* gu_s, int gs_gu,
                             const void* dn_w, const void* dn_s, int gs_dn, const void* tile_expert,
                             const void* tile_row0, const void* tile_rows, const void* tile_count,
                             int mtiles_max, const void* shared, void* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (T < 1 || k < 1 || E < 1 || H < BK || (H % BK) || (H % 8) || MI < BK || (MI % BK) ||
      gs_gu < BK || (gs_gu % BK) || (H % gs_gu) || gs_dn < BK || (gs_dn % BK) || (MI % gs_dn) ||
      !aligned16(x) || tile_expert == nullptr)
    return QMOE_EINVAL;
  if (workspace_bytes < qmoe_moe_prefill_workspace(T, k, H, MI)) return QMOE_EWORKSPACE;
  const int R = T * k;
  uint16_t* act = (uint16_t*)workspace;
  uint16_t* prod = (uint16_t*)((char*)workspace + (((size_t)R * MI * 2 + 255) & ~(size_t)255));
  hipStream_t st = (hipStream_t)stream;
  GemmArgs a{};
  a.a = (const uint16_t*)x; a.lda = H; a.perm = (const int64_t*)order; a.topk = k;
  a.w = (const uint32_t*)gu_w; a.s = (const uint16_t*)gu_s; a.K = H; a.N = 2 * MI; a.gs = gs_gu;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(MI, 64); a.y = act; a.ldy = MI; a.MI = MI;
  int rc = launch_gemm<1>(a, mtiles_max, st);
  if (rc) return rc;
  GemmArgs d = a;
  d.a = act; d.lda = MI; d.perm = (const int64_t*)order; d.topk = k;
  d.w = (const uint32_t*)dn_w; d.s = (const uint16_t*)dn_s; d.K = MI; d.N = H; d.gs = gs_dn;
  d.n_ntiles = host_ceil_div(H, BN); d.y = prod; d.ldy = H; d.wts = (const uint16_t*)wts;
  rc = launch_gemm<2>(d, mtiles_max, st);
  if (rc) return rc;
  hipLaunchKernelGGL(slot_reduce_kernel, dim3(host_ceil_div(H / 2, 256), T), dim3(256), 0, st, prod, T, k, H,
                     (const uint16_t*)shared, (uint16_t*)out);
  return (int)hipGetLastError();
}

}  // extern "C"
