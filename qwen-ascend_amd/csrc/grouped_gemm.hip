// Expert-major grouped W4A16 GEMM on MFMA (gfx950), for prefill.
//
//   y[p, n] = bf16( sum_k a[p, k] * q[e_p, k, n] * S[e_p, k / gs, n] )
//
// Rows p are sorted by expert; a row-tile table (expert, first row, rows)
// built on the GPU by the routing scan drives the grid, so empty experts cost
// nothing and no host synchronisation is needed.
//
// Exact fp16 operands. q (-8..7, <= 3 significant bits) times a bf16 scale
// (8 significant bits) needs at most 11 significant bits, so q*S is exactly
// representable in fp16 once the scales of a column are brought into fp16's
// range by a power of two: S' = S * 2^ec, max_g |S'| in [16, 32). A bf16
// activation is exact in fp16 after a per-row power of two: a' = a * 2^er,
// max_k |a'| in [2^13, 2^14). Every product a'*q*S' is then exact in fp32,
// the MFMA accumulates in fp32, and the epilogue removes 2^-(er+ec) exactly.
// The per-group scale is folded into the dequantised weight, so there is no
// per-group work on the accumulators.
//
// Dequantisation. Each lane owns one int32 word-column (8 output columns)
// and 8 consecutive k rows of it per MFMA step (its MFMA k-block). Row pairs
// are byte-interleaved with v_perm, each nibble pair becomes fp16 1 + u/16
// (u = q+8, in the top mantissa bits) with a shift and an and-or, and one
// v_pk_fma_f16 gives (1 + u/16) * 16S' - 1.5 * 16S' = q*S' for two rows at
// once (16S' and 1.5*16S' have at most 9 significant bits: both exact, and
// the fused result q*S' is exact). A lane thus feeds 8 MFMAs (one per column of
// its word), 16 lanes cover 16 word-columns = 128 output columns per wave.
//
// Tile: up to 128 rows (8 MFMA row tiles; tiles past the expert's rows are
// skipped) x 512 columns (4 waves x 128) per workgroup, K step 32. A rows
// (gathered through an optional permutation) are converted to fp16 into a
// double-buffered LDS chunk of 64 k; B words stream straight from HBM into
// registers one chunk (two steps) ahead.
//
// Epilogues: 0 = store bf16 rows; 1 = SwiGLU (gate word-columns in lanes
// 0..7, the matching up word-columns in lanes 8..15, swapped with DPP),
// writing act and the per-row max |act| for the next GEMM's row exponents;
// 2 = down projection with the top-k weight folded in:
// prod[order[p], n] = bf16(bf16(y) * w[order[p]]), scattered to token-major
// rows for the ordered slot reduction.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int BM = 128;          // rows per tile
constexpr int MT = BM / 16;      // MFMA row tiles
constexpr int BK = 32;           // k per MFMA step
constexpr int KC = 64;           // k per staged A chunk
constexpr int WAVE_COLS = 128;   // output columns per wave (16 word-columns)
constexpr int NC = 3;            // ring slots of 64-k chunks in LDS (two chunks in flight)
constexpr int BWORDS = 64;       // int32 word-columns of B per workgroup tile
constexpr int A_SLOT = BM * KC * 2;       // 16 KB: A fp16 [128][64]
constexpr int B_SLOT = KC * BWORDS * 4;   // 16 KB: B words [64][64]
constexpr int MAX_GROUPS = 56;            // scale rows staged in LDS (1 KB each)

struct GemmArgs {
  const _Float16* a16;       // fp16 activations (row-scaled by 2^rexp), row stride lda
  int lda;
  const int64_t* perm;       // mode 1: a row of p = perm[p] / topk; mode 2: output row of p = perm[p]
  int topk;
  const int* rexp;           // per a-row exponent, indexed like the a row
  uint32_t* rmax_out;        // mode 1: per row max |act| (bf16 bits), atomicMax
  const uint32_t* w;         // int4pack [E, K, N/8]
  const uint16_t* s;         // bf16 scales [E, G, N]
  int K, N, gs;
  const int* tile_expert;    // row-tile table (nullptr: dense, one expert, R rows)
  const int* tile_row0;
  const int* tile_rows;
  const int* tile_count;
  int R;
  int n_ntiles;
  uint16_t* y;
  int ldy;
  int MI;                    // mode 1: act width
  const uint16_t* wts;       // mode 2: bf16 routing weights, flat [T*topk]
};

QMOE_DEV half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
QMOE_DEV uint32_t h2_bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }
QMOE_DEV uint32_t pk_rtz(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// exponent that brings a magnitude with bf16 biased exponent eb into [2^t, 2^(t+1)), t = target - 127
QMOE_DEV int exp_to(uint32_t max_abs_bits, int target_biased) {
  const int eb = (int)(max_abs_bits >> 7) & 0xff;
  return eb == 0 ? 0 : target_biased - eb;
}

typedef float f32x8_t __attribute__((ext_vector_type(8)));

// s_waitcnt with vmcnt <= N and lgkmcnt == 0 (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4] left at 7).
template <int N>
QMOE_DEV void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4));
}

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte LDS read the compiler does not track. The compiler cannot tell
// which LDS bytes an in-flight global->LDS DMA writes, so it would wait for
// every outstanding DMA before an ordinary LDS read; this is used only for
// data whose DMA the caller has already waited for.
QMOE_DEV u32x4_t lds_read16_settled(const void* p) {
  u32x4_t v;
  const unsigned addr = (unsigned)(size_t)(const __attribute__((address_space(3))) char*)p;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
  return v;
}

// Workgroup barrier without a memory fence: the caller has already waited
// for the memory operations the barrier must order (a fence here would also
// wait for the B prefetches still in flight).
QMOE_DEV void barrier_no_fence() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// SwiGLU of 8 consecutive act columns of one row: act = bf16(silu(bf16(g)) *
// bf16(u)); stores them when `writer` and returns the row's max |act| bits
// over the gate lanes of the 16-lane row (every lane of the wave calls this).
__device__ __noinline__ uint32_t swiglu_store8(f32x8_t gv, f32x8_t uv, uint16_t* dst, bool writer) {
  uint32_t packed[4], amax = 0;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const uint32_t a0 = f32_to_bf16(silu_f32(round_bf16(gv[j])) * round_bf16(uv[j]));
    const uint32_t a1 = f32_to_bf16(silu_f32(round_bf16(gv[j + 1])) * round_bf16(uv[j + 1]));
    packed[j >> 1] = a0 | (a1 << 16);
    amax = max(amax, max(a0 & 0x7fffu, a1 & 0x7fffu));
  }
  if (writer) *reinterpret_cast<uint4*>(dst) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  amax = writer ? amax : 0u;
  amax = max(amax, (uint32_t)__builtin_amdgcn_update_dpp((int)amax, (int)amax, 0xB1, 0xf, 0xf, false));
  amax = max(amax, (uint32_t)__builtin_amdgcn_update_dpp((int)amax, (int)amax, 0x4E, 0xf, 0xf, false));
  amax = max(amax, (uint32_t)__builtin_amdgcn_update_dpp((int)amax, (int)amax, 0x141, 0xf, 0xf, false));
  return amax;
}

// fp16 pair (1 + u_lo/16, 1 + u_hi/16) from nibble J of both 16-bit halves
// of t: the nibble goes to mantissa bits 6..9 under exponent 0.
template <int J>
QMOE_DEV uint32_t magic_pair(uint32_t t) {
  const uint32_t sh = (J == 0) ? (t << 6) : (J == 1) ? (t << 2) : (J == 2) ? (t >> 2) : (t >> 6);
  return (sh & 0x03C003C0u) | 0x3C003C00u;
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void grouped_gemm_f16_kernel(GemmArgs g) {
  // LDS: a ring of NC chunks (A fp16 [128 rows][64 k], XOR-swizzled by 16-byte
  // chunk; B int4 words [64 k][64 word-columns]), then the scale rows of all
  // groups for the workgroup's 64 word-columns, then per-row exponents.
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  unsigned char* As_base = lds;                                   // NC * 16 KB
  unsigned char* Bs_base = lds + NC * A_SLOT;                     // NC * 16 KB
  unsigned char* Ss = lds + NC * (A_SLOT + B_SLOT);              // G * 1 KB
  int* s_erow = reinterpret_cast<int*>(Ss + (size_t)(g.K / g.gs) * 1024);

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
  const int i16 = lane & 15;
  const int kb = lane >> 4;  // MFMA k-block of this lane (rows 8kb..8kb+7 of a step)
  const int K = g.K, N = g.N, nw = N >> 3;
  const int G = K / g.gs;
  const int nch = K / KC;

  // ---- the workgroup's 64 word-columns: global word-column of tile column c
  auto tile_word = [&](int c, bool& ok) -> int {
    if (MODE == 1) {
      const int a = nt * 256 + 8 * (c & 31);  // act column of the word
      ok = a < g.MI;
      return ok ? (((c < 32) ? a : g.MI + a) >> 3) : 0;
    }
    const int col = nt * 512 + 8 * c;
    ok = col < N;
    return ok ? (col >> 3) : 0;
  };
  // this lane's tile column and output columns
  const int tcol = (MODE == 1) ? ((i16 < 8) ? 8 * wave + i16 : 32 + 8 * wave + (i16 - 8)) : 16 * wave + i16;
  bool col_ok;
  (void)tile_word(tcol, col_ok);
  const int outcol0 = (MODE == 1) ? nt * 256 + 8 * (8 * wave + (i16 & 7)) : nt * 512 + 8 * tcol;

  const uint32_t* we = g.w + (size_t)e * K * nw;
  const uint16_t* se = g.s + (size_t)e * G * N;

  // ---- DMA sources. B: thread t, instruction q -> rows 4(4q+wave) + lane/16,
  // tile words 4(lane%16)..+3. A: instruction q -> rows 8(4q+wave) + lane/8,
  // LDS chunk lane%8 holding global k-chunk (lane%8) ^ (row & 7).
  const uint32_t* bsrc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    bool ok;
    const int w0 = tile_word(4 * (lane & 15), ok);
    const int r = 4 * (4 * q + wave) + (lane >> 4);
    bsrc[q] = we + (size_t)r * nw + w0;
  }
  const _Float16* asrc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = 8 * (4 * q + wave) + (lane >> 3);
    const int p = row0 + min(r, rows - 1);
    const int src = (MODE == 1 && g.perm != nullptr) ? (int)(g.perm[p] / g.topk) : p;
    const int c = (lane & 7) ^ (r & 7);
    asrc[q] = g.a16 + (size_t)src * g.lda + 8 * c;
  }
  auto issue_chunk = [&](int ch, int slot) {
    const int k0 = ch * KC;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      __builtin_amdgcn_global_load_lds(bsrc[q] + (size_t)k0 * nw, Bs_base + slot * B_SLOT + (4 * q + wave) * 1024, 16, 0, 0);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      __builtin_amdgcn_global_load_lds(asrc[q] + k0, As_base + slot * A_SLOT + (4 * q + wave) * 1024, 16, 0, 0);
  };

  // ---- prologue. Row exponents first (ordinary loads, consumed at once),
  // then the DMA: all scale rows (group gi by wave gi % 4), chunks 0 and 1.
  if (tid < BM) {
    const int r = tid;
    const int p = row0 + min(r, rows - 1);
    const int src = (MODE == 1 && g.perm != nullptr) ? (int)(g.perm[p] / g.topk) : p;
    s_erow[r] = (r < rows) ? g.rexp[src] : 0;
  }
  {
    bool ok;
    const int w = tile_word(lane, ok);
    const uint16_t* ssrc = se + (size_t)w * 8;
    for (int gi = wave; gi < G; gi += 4)
      __builtin_amdgcn_global_load_lds(ssrc + (size_t)gi * N, Ss + gi * 1024, 16, 0, 0);
  }
  issue_chunk(0, 0);
  if (nch > 1) issue_chunk(1, 1);
  // scales and chunk 0 have landed once only chunk 1 (8 DMA per thread) may be pending
  if (nch > 1) wait_vm_lgkm0<8>();
  else wait_vm_lgkm0<0>();
  barrier_no_fence();

  // column exponents: max over all groups of |S| of this lane's 8 columns
  int ec[8];
  {
    uint32_t mx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int gi = 0; gi < G; ++gi) {
      const u32x4_t v = lds_read16_settled(Ss + gi * 1024 + tcol * 16);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        mx[2 * q] = max(mx[2 * q], vv[q] & 0x7fffu);
        mx[2 * q + 1] = max(mx[2 * q + 1], (vv[q] >> 16) & 0x7fffu);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ec[j] = exp_to(mx[j], 131);
  }

  // scale pairs of the current group: (16S', 16S') and (-24S', -24S')
  uint32_t sp[8], sn[8];
  auto load_scales = [&](int grp) {
    const u32x4_t v = lds_read16_settled(Ss + grp * 1024 + tcol * 16);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t b = (j & 1) ? (vv[j >> 1] >> 16) : (vv[j >> 1] & 0xffffu);
      const float f = ldexpf(bf16_to_f32(b), ec[j] + 4);
      sp[j] = pk_rtz(f, f);
      sn[j] = pk_rtz(-1.5f * f, -1.5f * f);
    }
  };

  f32x4_t acc[MT][8];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[t][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int live = min(MT, (rows + 15) >> 4);
  const int steps_per_group = g.gs / BK;

  // one MFMA step: dequantise this lane's 8x8 nibble block into 8 fp16 B
  // fragments, then MFMA them against every live row tile
  auto mfma_step = [&](int slot, int half) {
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(Bs_base + slot * B_SLOT);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = bs[(32 * half + 8 * kb + i) * BWORDS + tcol];
    uint32_t tl[4], th[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
      tl[pr] = __builtin_amdgcn_perm(w[2 * pr + 1], w[2 * pr], 0x05040100u) ^ 0x88888888u;
      th[pr] = __builtin_amdgcn_perm(w[2 * pr + 1], w[2 * pr], 0x07060302u) ^ 0x88888888u;
    }
    half8_t bf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t h[4];
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        const uint32_t t = (j < 4) ? tl[pr] : th[pr];
        uint32_t m;
        switch (j & 3) {
          case 0: m = magic_pair<0>(t); break;
          case 1: m = magic_pair<1>(t); break;
          case 2: m = magic_pair<2>(t); break;
          default: m = magic_pair<3>(t); break;
        }
        h[pr] = h2_bits(__builtin_elementwise_fma(as_h2(m), as_h2(sp[j]), as_h2(sn[j])));
      }
      bf[j] = __builtin_bit_cast(half8_t, make_uint4(h[0], h[1], h[2], h[3]));
    }
    const unsigned char* as = As_base + slot * A_SLOT;
    const int kc = 4 * half + kb;  // 16-byte k-chunk of this lane's A fragment
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < live) {
        const int r = 16 * t + i16;
        const half8_t af = *reinterpret_cast<const half8_t*>(as + r * 128 + ((kc ^ (r & 7)) << 4));
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[t][j], 0, 0, 0);
      }
    }
  };

  for (int c = 0; c < nch; ++c) {
    if (c > 0) {
      // chunk c has landed once only chunk c+1 (8 DMA per thread) may be pending
      if (c + 1 < nch) wait_vm_lgkm0<8>();
      else wait_vm_lgkm0<0>();
      barrier_no_fence();
    }
    // every wave is past chunk c-1: its ring slot takes chunk c+2
    if (c + 2 < nch) issue_chunk(c + 2, (c + 2) % NC);
    const int slot = c % NC;
    if ((2 * c) % steps_per_group == 0) load_scales((2 * c) / steps_per_group);
    mfma_step(slot, 0);
    if ((2 * c + 1) % steps_per_group == 0) load_scales((2 * c + 1) / steps_per_group);
    mfma_step(slot, 1);
  }

  // ---- epilogue. MFMA 16x16 layout: lane holds column (word i16, nibble j)
  // of rows 4*kb + r, r = 0..3, of each row tile.
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    if (t >= live) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * t + 4 * kb + r;
      const bool ok = row < rows && col_ok;
      const int p = row0 + min(row, rows - 1);
      const int er = s_erow[row];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = ldexpf(acc[t][j][r], -(er + ec[j]));
      if (MODE == 1) {
        // up values live in lanes i16 + 8 of the same 16-lane row
        f32x8_t gv, uv;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          gv[j] = v[j];
          uv[j] = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v[j]), __float_as_int(v[j]), 0x108, 0xf, 0xf, false));
        }
        const uint32_t amax = swiglu_store8(gv, uv, g.y + (size_t)p * g.ldy + outcol0, ok && i16 < 8);
        if (i16 == 0 && row < rows) atomicMax(g.rmax_out + p, amax);
      } else if (MODE == 2) {
        if (ok) {
          const int64_t f = g.perm[p];
          const float wv2 = bf16_to_f32(g.wts[f]);
          uint32_t packed[4];
#pragma unroll
          for (int j = 0; j < 8; j += 2)
            packed[j >> 1] = f32_to_bf16(round_bf16(v[j]) * wv2) | (f32_to_bf16(round_bf16(v[j + 1]) * wv2) << 16);
          *reinterpret_cast<uint4*>(g.y + (size_t)f * g.ldy + outcol0) =
              make_uint4(packed[0], packed[1], packed[2], packed[3]);
        }
      } else {
        if (ok) {
          uint32_t packed[4];
#pragma unroll
          for (int j = 0; j < 8; j += 2) packed[j >> 1] = f32_to_bf16(v[j]) | (f32_to_bf16(v[j + 1]) << 16);
          *reinterpret_cast<uint4*>(g.y + (size_t)p * g.ldy + outcol0) =
              make_uint4(packed[0], packed[1], packed[2], packed[3]);
        }
      }
    }
  }
}

// Per-row exponent and fp16 copy of bf16 rows: e = exponent that puts
// max |x| * 2^e in [2^13, 2^14), x16 = fp16(x * 2^e) (exact: a bf16 value
// keeps its 8 significant bits). One wave per row; `rmax` (optional) gives
// the row maxima instead of a scan. Also clears an optional buffer of
// `nzero` words.
__global__ __launch_bounds__(256) void rows_to_f16_kernel(const uint16_t* __restrict__ x, int rows, int K,
                                                          const uint32_t* __restrict__ rmax, int* __restrict__ rexp,
                                                          _Float16* __restrict__ x16, uint32_t* __restrict__ zero,
                                                          int nzero) {
  const int gtid = blockIdx.x * 256 + threadIdx.x;
  for (int q = gtid; q < nzero; q += gridDim.x * 256) zero[q] = 0u;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* xr = x + (size_t)row * K;
  uint32_t m = 0;
  if (rmax != nullptr) {
    m = rmax[row];
  } else {
    for (int c = lane * 8; c < K; c += 512) {
      const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) m = max(m, max(vv[q] & 0x7fffu, (vv[q] >> 16) & 0x7fffu));
    }
    m = wave_max_u32(m);
  }
  const int e = exp_to(m, 140);
  if (lane == 0) rexp[row] = e;
  const float sc = ldexpf(1.0f, e);
  _Float16* yr = x16 + (size_t)row * K;
  for (int c = lane * 8; c < K; c += 512) {
    const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      h[q] = pk_rtz(__uint_as_float(vv[q] << 16) * sc, __uint_as_float(vv[q] & 0xffff0000u) * sc);
    *reinterpret_cast<uint4*>(yr + c) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

// out[t, n] = bf16(sum_{j < k, in order} prod[t*k + j, n]) (+ shared, a bf16 add)
__global__ __launch_bounds__(256) void slot_reduce_kernel(const uint16_t* __restrict__ prod, int T, int k, int H,
                                                          const uint16_t* __restrict__ shared,
                                                          uint16_t* __restrict__ out) {
  const int c8 = blockIdx.x * 256 + threadIdx.x;  // group of 8 columns
  if (8 * c8 >= H) return;
  for (int t = blockIdx.y; t < T; t += gridDim.y) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < k; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(prod + ((size_t)t * k + j) * H + 8 * c8);
      const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a[2 * q] += bf16_to_f32(vv[q] & 0xffffu);
        a[2 * q + 1] += bf16_to_f32(vv[q] >> 16);
      }
    }
    uint32_t r[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = f32_to_bf16(a[q]);
    if (shared != nullptr) {
      const uint4 sv = *reinterpret_cast<const uint4*>(shared + (size_t)t * H + 8 * c8);
      const uint32_t ss[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        r[2 * q] = f32_to_bf16(bf16_to_f32(r[2 * q]) + bf16_to_f32(ss[q] & 0xffffu));
        r[2 * q + 1] = f32_to_bf16(bf16_to_f32(r[2 * q + 1]) + bf16_to_f32(ss[q] >> 16));
      }
    }
    *reinterpret_cast<uint4*>(out + (size_t)t * H + 8 * c8) =
        make_uint4(r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16), r[6] | (r[7] << 16));
  }
}

size_t gemm_lds_bytes(int G) { return (size_t)NC * (A_SLOT + B_SLOT) + (size_t)G * 1024 + BM * sizeof(int); }

template <int MODE>
int launch_gemm(const GemmArgs& a, int mtiles_max, hipStream_t st) {
  const long nblk = (long)mtiles_max * a.n_ntiles;
  if (nblk <= 0) return 0;
  const size_t lds = gemm_lds_bytes(a.K / a.gs);
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute((const void*)grouped_gemm_f16_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)gemm_lds_bytes(MAX_GROUPS));
    attr_set = true;
  }
  hipLaunchKernelGGL((grouped_gemm_f16_kernel<MODE>), dim3((unsigned)nblk), dim3(kThreads), lds, st, a);
  return (int)hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launch_rows_to_f16(const void* x, int rows, int K, const uint32_t* rmax, int* rexp, _Float16* x16,
                       uint32_t* zero, int nzero, hipStream_t st) {
  const int blocks = max(host_ceil_div(rows, 4), host_ceil_div(nzero, 256));
  hipLaunchKernelGGL(rows_to_f16_kernel, dim3(max(blocks, 1)), dim3(256), 0, st, (const uint16_t*)x, rows, K, rmax,
                     rexp, x16, zero, nzero);
  return (int)hipGetLastError();
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

bool gemm_shape_ok(int K, int N, int gs) {
  return K >= KC && K % KC == 0 && N >= 8 && N % 8 == 0 && gs >= BK && gs % BK == 0 && K % gs == 0 &&
         K / gs <= MAX_GROUPS;
}

// workspace of a plain GEMM: fp16 rows [R, K] | row exponents [R]
size_t plain_ws(int R, int K) { return align256((size_t)R * K * 2) + align256((size_t)R * 4); }

// workspace of the fused prefill:
//   act [R, MI] bf16 | act16 [R, MI] fp16 | prod [R, H] bf16 | x16 [T, H] fp16 |
//   x row exponents [T] | act row max [R] | act row exponents [R]
struct PrefillLayout {
  size_t act, act16, prod, x16, rexp_x, rmax, rexp_a, total;
};
PrefillLayout prefill_layout(int T, int k, int H, int MI) {
  const size_t R = (size_t)T * k;
  PrefillLayout l;
  size_t o = 0;
  l.act = o; o += align256(R * MI * 2);
  l.act16 = o; o += align256(R * MI * 2);
  l.prod = o; o += align256(R * H * 2);
  l.x16 = o; o += align256((size_t)T * H * 2);
  l.rexp_x = o; o += align256((size_t)T * 4);
  l.rmax = o; o += align256(R * 4);
  l.rexp_a = o; o += align256(R * 4);
  l.total = o;
  return l;
}

}  // namespace

// ============================================================================ C ABI

extern "C" {

int qmoe_gemm_tile_rows(void) { return BM; }

size_t qmoe_grouped_gemm_workspace(int R, int K) { return plain_ws(R > 0 ? R : 1, K); }

int qmoe_grouped_gemm(const void* x, int R, int K, int N, int E, int gs, const void* w, const void* scale,
                      const void* tile_expert, const void* tile_row0, const void* tile_rows,
                      const void* tile_count, int mtiles_max, void* y, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (R < 0 || E < 1 || !gemm_shape_ok(K, N, gs) || !aligned16(x) || !aligned16(y) || !aligned16(scale) ||
      !aligned16(workspace) || tile_expert == nullptr)
    return QMOE_EINVAL;
  if (R == 0) return 0;
  if (workspace_bytes < qmoe_grouped_gemm_workspace(R, K)) return QMOE_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  _Float16* x16 = (_Float16*)workspace;
  int* rexp = (int*)((char*)workspace + align256((size_t)R * K * 2));
  int rc = launch_rows_to_f16(x, R, K, nullptr, rexp, x16, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a16 = x16; a.lda = K; a.perm = nullptr; a.topk = 1; a.rexp = rexp;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(N, 512); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, mtiles_max, st);
}

size_t qmoe_w4a16_gemm_mfma_workspace(int M, int K) { return plain_ws(M > 0 ? M : 1, K); }

int qmoe_w4a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int gs,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 1 || !gemm_shape_ok(K, N, gs) || !aligned16(x) || !aligned16(y) || !aligned16(scale) ||
      !aligned16(workspace))
    return QMOE_EINVAL;
  if (workspace_bytes < qmoe_w4a16_gemm_mfma_workspace(M, K)) return QMOE_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  _Float16* x16 = (_Float16*)workspace;
  int* rexp = (int*)((char*)workspace + align256((size_t)M * K * 2));
  int rc = launch_rows_to_f16(x, M, K, nullptr, rexp, x16, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a16 = x16; a.lda = K; a.topk = 1; a.rexp = rexp;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.R = M; a.n_ntiles = host_ceil_div(N, 512); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, host_ceil_div(M, BM), st);
}

size_t qmoe_moe_prefill_workspace(int T, int k, int H, int MI) { return prefill_layout(T, k, H, MI).total; }

int qmoe_moe_prefill_layout(int T, int k, int H, int MI, size_t* off_act, size_t* off_prod) {
  if (T < 1 || k < 1 || H < 1 || MI < 1 || off_act == nullptr || off_prod == nullptr) return QMOE_EINVAL;
  const PrefillLayout l = prefill_layout(T, k, H, MI);
  *off_act = l.act;
  *off_prod = l.prod;
  return 0;
}

int qmoe_moe_experts_grouped(const void* x, int T, int H, int MI, int E, int k, const void* wts,
                             const void* order, const void* gu_w, const void* gu_s, int gs_gu,
                             const void* dn_w, const void* dn_s, int gs_dn, const void* tile_expert,
                             const void* tile_row0, const void* tile_rows, const void* tile_count,
                             int mtiles_max, const void* shared, void* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (T < 1 || k < 1 || E < 1 || !gemm_shape_ok(H, 2 * MI, gs_gu) || !gemm_shape_ok(MI, H, gs_dn) ||
      !aligned16(x) || !aligned16(out) || !aligned16(gu_s) || !aligned16(dn_s) || !aligned16(workspace) ||
      (shared != nullptr && !aligned16(shared)) || tile_expert == nullptr)
    return QMOE_EINVAL;
  const PrefillLayout l = prefill_layout(T, k, H, MI);
  if (workspace_bytes < l.total) return QMOE_EWORKSPACE;
  const int R = T * k;
  char* ws = (char*)workspace;
  uint16_t* act = (uint16_t*)(ws + l.act);
  _Float16* act16 = (_Float16*)(ws + l.act16);
  uint16_t* prod = (uint16_t*)(ws + l.prod);
  _Float16* x16 = (_Float16*)(ws + l.x16);
  int* rexp_x = (int*)(ws + l.rexp_x);
  uint32_t* rmax = (uint32_t*)(ws + l.rmax);
  int* rexp_a = (int*)(ws + l.rexp_a);
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_rows_to_f16(x, T, H, nullptr, rexp_x, x16, rmax, R, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a16 = x16; a.lda = H; a.perm = (const int64_t*)order; a.topk = k; a.rexp = rexp_x; a.rmax_out = rmax;
  a.w = (const uint32_t*)gu_w; a.s = (const uint16_t*)gu_s; a.K = H; a.N = 2 * MI; a.gs = gs_gu;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(MI, 256); a.y = act; a.ldy = MI; a.MI = MI;
  rc = launch_gemm<1>(a, mtiles_max, st);
  if (rc) return rc;
  rc = launch_rows_to_f16(act, R, MI, rmax, rexp_a, act16, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs d = a;
  d.a16 = act16; d.lda = MI; d.perm = (const int64_t*)order; d.topk = k; d.rexp = rexp_a; d.rmax_out = nullptr;
  d.w = (const uint32_t*)dn_w; d.s = (const uint16_t*)dn_s; d.K = MI; d.N = H; d.gs = gs_dn;
  d.n_ntiles = host_ceil_div(H, 512); d.y = prod; d.ldy = H; d.wts = (const uint16_t*)wts;
  rc = launch_gemm<2>(d, mtiles_max, st);
  if (rc) return rc;
  hipLaunchKernelGGL(slot_reduce_kernel, dim3(host_ceil_div(H / 8, 256), min(T, 65535)), dim3(256), 0, st, prod, T,
                     k, H, (const uint16_t*)shared, (uint16_t*)out);
  return (int)hipGetLastError();
}

}  // extern "C"
