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
// Dequantisation. A lane owns 8 consecutive k rows (its MFMA k-block) of one
// or two int32 words per MFMA step. Row pairs are byte-interleaved with
// v_perm, a nibble pair becomes fp16 1 + u/16 (u = q+8, in the top mantissa
// bits) with a shift and one v_bitop3 (mask, flip of the nibble's top bit,
// exponent bits), and one v_pk_fma_f16 gives
// (1 + u/16) * 16S' - 1.5 * 16S' = q*S' for two rows at once (16S' and
// 1.5*16S' have at most 9 significant bits: both exact, and the fused result
// q*S' is exact). Each lane feeds four 16x16x32 MFMA B fragments per step.
//
// Tile: up to 128 rows (8 MFMA row tiles; tiles past the expert's rows are
// skipped) x 32 int32 word-columns (256 output or 128 SwiGLU columns) per
// workgroup of 4 waves; two workgroups per CU give two waves per SIMD, so
// one wave's dequantisation runs beside the other's MFMA. Wave w owns tile
// words 8w..8w+7, lane i taking nibbles 4(i/8)..+3 of word i%8 (mode 1: words
// 8w..8w+3 are the gate words of act words 4w..4w+3 and 8w+4..8w+7 their up
// words, so the up value of a gate lane sits 4 lanes up, one DPP shift away). A (fp16 rows, gathered through the permutation in mode 1),
// B (int4 words) and the bf16 scale rows of the chunk's groups stream
// through a ring of three 64-k LDS chunks by buffer-resource global->LDS
// DMA, two chunks ahead. Real row tiles are spread over the 8 XCDs.
//
// Epilogues: 0 = store bf16 rows; 1 = SwiGLU, writing act and the per-row
// max |act| for the next GEMM's row exponents; 2 = down projection with the
// top-k weight folded in: prod[order[p], n] = bf16(bf16(y) * w[order[p]]),
// scattered to token-major rows for the ordered slot reduction.
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;    // 4 waves; two workgroups per CU, so two waves per SIMD
constexpr int BM = 128;          // rows per tile
constexpr int MT = BM / 16;      // MFMA row tiles
constexpr int BK = 32;           // k per MFMA step
constexpr int KC = 64;           // k per staged chunk
constexpr int NC = 3;            // ring slots of 64-k chunks in LDS (two chunks in flight)
constexpr int BWORDS = 32;       // int32 word-columns of B per workgroup tile
constexpr int A_SLOT = BM * KC * 2;       // 16 KB: A fp16 [128][64]
constexpr int B_SLOT = KC * BWORDS * 4;   // 8 KB: B words [64][32]
constexpr int S_SLOT = 2 * BWORDS * 16;   // 1 KB: bf16 scales of the groups of the chunk's two steps
constexpr int SLOT = A_SLOT + B_SLOT + S_SLOT;

struct GemmArgs {
  const _Float16* a16;       // fp16 activations (row-scaled by 2^rexp), row stride lda
  int lda;
  uint32_t a_bytes;          // extent of a16 in bytes (< 2^31)
  const int64_t* perm;       // mode 1: a row of p = perm[p] / topk; mode 2: output row of p = perm[p] (both required)
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
  int mtiles_max;            // row tiles the grid was sized for (tile_count is clamped to it)
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
// bf16 pair (RNE, hardware conversion; finite values round exactly like f32_to_bf16)
QMOE_DEV uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
QMOE_DEV float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
QMOE_DEV float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// exponent that brings a magnitude with bf16 biased exponent eb into [2^t, 2^(t+1)), t = target - 127
QMOE_DEV int exp_to(uint32_t max_abs_bits, int target_biased) {
  const int eb = (int)(max_abs_bits >> 7) & 0xff;
  return eb == 0 ? 0 : target_biased - eb;
}

// s_waitcnt with vmcnt <= N and lgkmcnt == 0 (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4] left at 7).
template <int N>
QMOE_DEV void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4));
}

// LDS accesses the compiler does not track. The compiler cannot tell which
// LDS bytes an in-flight global->LDS DMA writes, so it would wait for every
// outstanding DMA before an ordinary LDS access; these are used only for data
// that no DMA in flight touches. Reads wait for their own result.
QMOE_DEV unsigned lds_addr(const void* p) {
  return (unsigned)(size_t)(const __attribute__((address_space(3))) char*)p;
}
QMOE_DEV u32x4_t lds_read16_settled(const void* p) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
QMOE_DEV u32x2_t lds_read8_settled(const void* p) {
  u32x2_t v;
  asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
QMOE_DEV uint32_t lds_read4_settled(const void* p) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
QMOE_DEV void lds_write16_settled(void* p, u32x4_t v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}
QMOE_DEV void lds_write4_settled(void* p, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}
QMOE_DEV void lds_max4_settled(void* p, uint32_t v) {
  asm volatile("ds_max_u32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}

// Workgroup barrier without a memory fence: the caller has already waited
// for the memory operations the barrier must order (a fence here would also
// wait for the prefetches still in flight).
QMOE_DEV void barrier_no_fence() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// A constant held in a VGPR the compiler cannot see through, so that the
// loop keeps it in a register and uses three-operand forms (v_and_or_b32)
// instead of two instructions with literals.
QMOE_DEV uint32_t opaque_vreg(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

// DPP max over the 16 lanes of a row
QMOE_DEV uint32_t row16_max(uint32_t v) {
  v = max(v, QMOE_DPP(v, 0xB1));   // quad_perm [1,0,3,2]
  v = max(v, QMOE_DPP(v, 0x4E));   // quad_perm [2,3,0,1]
  v = max(v, QMOE_DPP(v, 0x141));  // row_half_mirror
  v = max(v, QMOE_DPP(v, 0x140));  // row_mirror
  return v;
}

// fp16 pair (1 + u_lo/16, 1 + u_hi/16) from nibble J of both 16-bit halves
// of t: the nibble goes to mantissa bits 6..9 under exponent 0.
template <int J>
QMOE_DEV uint32_t magic_pair(uint32_t t, uint32_t mask, uint32_t one) {
  const uint32_t sh = (J == 0) ? (t << 6) : (J == 1) ? (t << 2) : (J == 2) ? (t >> 2) : (t >> 6);
  return (sh & mask) | one;
}
// the same with the nibble chosen per lane: rotate right by 26, 30, 2, 6
// for nibble 0, 1, 2, 3 (the bits that wrap around fall outside the mask)
QMOE_DEV uint32_t magic_pair_rot(uint32_t t, uint32_t rot, uint32_t mask, uint32_t one) {
  return (__builtin_amdgcn_alignbit(t, t, rot) & mask) | one;
}
// scale pair (s, s) from the low or high fp16 of v
QMOE_DEV uint32_t dup_lo(uint32_t v) { return __builtin_amdgcn_perm(v, v, 0x01000100u); }
QMOE_DEV uint32_t dup_hi(uint32_t v) { return __builtin_amdgcn_perm(v, v, 0x03020302u); }
QMOE_DEV uint32_t times_m15(uint32_t v) {
  const half2_t m15 = {(_Float16)-1.5f, (_Float16)-1.5f};
  return h2_bits(as_h2(v) * m15);
}

template <int N>
struct IntC {
  static constexpr int value = N;
};

template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void grouped_gemm_f16_kernel(GemmArgs g) {
  // LDS: a ring of NC chunks, each B (int4 words [64 k][32 word-columns],
  // XOR-swizzled by k-block), A (fp16 [128 rows][64 k], XOR-swizzled by
  // 16-byte chunk) and the raw bf16 scale rows of the groups of its two
  // steps; then the per-column max |S| and per-row data. About 78 KB, so two
  // workgroups share a CU and their waves pair up on each SIMD.
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int G = g.K / g.gs;
  uint32_t* s_mx = reinterpret_cast<uint32_t*>(lds + NC * SLOT);   // [32 words][8 columns]
  int* s_erow = reinterpret_cast<int*>(s_mx + 256);                 // [BM] row exponents
  int* s_orow = s_erow + BM;                                        // [BM] mode 2: output row
  float* s_wrow = reinterpret_cast<float*>(s_orow + BM);            // [BM] mode 2: routing weight
  uint32_t* s_rmax = reinterpret_cast<uint32_t*>(s_wrow + BM);      // [BM] mode 1: row max |act|

  // ---- tile of this block. Block b runs on XCD b % 8 and is the (b / 8)-th
  // block of its XCD: XCD x takes row tiles x, x + 8, x + 16, ... in table
  // order (the table lists them longest first), each with all its column
  // tiles in a row, which share their A rows through the XCD's L2.
  const int tiles_m = (g.tile_expert != nullptr) ? min(g.tile_count[0], g.mtiles_max) : ceil_div(g.R, BM);
  const int xi = (int)(blockIdx.x >> 3);
  const int rt_local = xi / g.n_ntiles;
  const int nt = xi - rt_local * g.n_ntiles;
  const int mt = 8 * rt_local + (int)(blockIdx.x & 7);
  if (mt >= tiles_m) return;
  int e, row0, rows;
  if (g.tile_expert != nullptr) {
    e = g.tile_expert[mt];
    row0 = g.tile_row0[mt];
    rows = g.tile_rows[mt];
  } else {
    e = 0;
    row0 = mt * BM;
    rows = min(BM, g.R - row0);
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int i16 = lane & 15;
  const int kb = lane >> 4;  // MFMA k-block of this lane (rows 8kb..8kb+7 of a step)
  const int K = g.K, N = g.N, nw = N >> 3;
  const int nch = K / KC;

  // ---- the workgroup's 32 word-columns. Mode 0/2: tile column c is word
  // nt*32 + c. Mode 1: tile column c of wave c/8 is the gate word ((c%8) < 4)
  // or the up word of act word 4(c/8) + c%4.
  auto tile_word = [&](int c, bool& ok) -> int {
    if (MODE == 1) {
      const int a = nt * 128 + 8 * (4 * (c >> 3) + (c & 3));  // act column of the word
      ok = a < g.MI;
      return ok ? ((((c & 7) < 4) ? a : g.MI + a) >> 3) : 0;
    }
    const int col = nt * 256 + 8 * c;
    ok = col < N;
    return ok ? (col >> 3) : 0;
  };
  // this lane's word and output columns: nibbles 4hi..4hi+3 of tile word
  // tc_a (mode 1: the act columns of a gate lane)
  const int hi = i16 >> 3;
  const int tc_a = 8 * wave + (i16 & 7);
  bool col_ok;
  (void)tile_word(tc_a, col_ok);
  const int outcol = (MODE == 1) ? nt * 128 + 8 * (4 * wave + (i16 & 3)) + 4 * hi : nt * 256 + 8 * tc_a + 4 * hi;

  const uint32_t* we = g.w + (size_t)e * K * nw;
  const uint16_t* se = g.s + (size_t)e * G * N;

  // ---- DMA sources, per chunk and thread: 2 B, NQ = ceil(LIVE/2) A and 1
  // scale instruction.
  // B: instruction q -> 1 KB block 4q+wave = k-rows 8(4q+wave) + lane/8, LDS
  // word positions 4(lane%8)..+3 holding tile columns (position ^ 8*wave):
  // the swizzle 8 * ((k-row / 8) % 4) puts the four k-blocks a wave reads at
  // once in different banks. A: instruction q -> row group
  // gi = min(4q+wave, 2*LIVE-1), rows 8gi + lane/8, LDS chunk lane%8 holding
  // global k-chunk (lane%8) ^ (row & 7); only the live row tiles are fetched
  // (a group past them re-fetches the last live group, same bytes to the same
  // place). Scales:
  // lane l < 16 of wave w, the row of the group of step l/8 for tile word
  // 8w + l%8, at [w][step][word % 8][8 columns].
  // DMA through buffer resources: a wave-uniform SGPR offset advanced per
  // chunk plus a per-lane VGPR offset fixed for the whole loop, so the loop
  // spends no vector instructions on addresses. The resources also bound
  // every access to its tensor.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  constexpr int kRsrcWord3 = 0x00020000;
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void*)we, (short)0, K * nw * 4, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_s = __builtin_amdgcn_make_buffer_rsrc((void*)se, (short)0, G * N * 2, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc((void*)g.a16, (short)0, (int)g.a_bytes, kRsrcWord3);
  uint32_t boff, soff, aoff[4] = {0u, 0u, 0u, 0u};
  {
    bool ok;
    boff = 4u * (uint32_t)((lane >> 3) * nw + tile_word((4 * (lane & 7)) ^ (8 * wave), ok));
    soff = 2u * 8u * (uint32_t)tile_word(8 * wave + (lane & 7), ok);
  }
  auto issue_chunk = [&](auto live_c, int ch, int slot) {
    constexpr int LIVE = decltype(live_c)::value;
    unsigned char* base = lds + slot * SLOT;
    const int k0 = ch * KC;
#pragma unroll
    for (int q = 0; q < 2; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (__attribute__((address_space(3))) void*)(base + (4 * q + wave_u) * 1024), 16,
                                               (int)boff, (k0 + 8 * (4 * q + wave_u)) * nw * 4, 0, 0);
#pragma unroll
    for (int q = 0; q < (LIVE + 1) / 2; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a,
                                               (__attribute__((address_space(3))) void*)(base + B_SLOT + min(4 * q + wave_u, 2 * LIVE - 1) * 1024),
                                               16, (int)aoff[q], k0 * 2, 0, 0);
    // scale rows of the groups of the chunk's two steps (lanes 0..7: step 0,
    // lanes 8..15: step 1)
    const int g0 = k0 / g.gs, g1 = (k0 + BK) / g.gs;
    if (lane < 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_s, (__attribute__((address_space(3))) void*)(base + B_SLOT + A_SLOT + wave_u * 256), 16,
                                               (int)(soff + ((lane >> 3) ? (uint32_t)((g1 - g0) * N * 2) : 0u)), g0 * N * 2, 0, 0);
  };

  // Everything below is specialised on the live row-tile count, so that the
  // A DMA fetches only live rows and only live accumulators occupy registers.
  const int live = min(MT, (rows + 15) >> 4);
  auto body = [&](auto live_c) {
  constexpr int LIVE_B = decltype(live_c)::value;
  constexpr int NQ = (LIVE_B + 1) / 2;  // A DMA instructions per thread and chunk
  // ---- prologue. The A row indices first (mode 1: through the
  // permutation; entries are < 2^31, they index T*topk rows) and the
  // permutation entry of this thread's epilogue row (thread t: tile row
  // t % BM), then the DMA of chunks 0 and 1 as soon as their addresses are
  // known, then, while those land, the column maxima of |S| over all groups
  // (word tid%32, groups tid/32, tid/32 + 8, ...) and the per-row data, which
  // only the epilogue reads.
  // (the maxima's LDS words are cleared first: an asm LDS store after a
  // global load would wait for that load)
  lds_write4_settled(s_mx + tid, 0u);
  const int drow = tid & (BM - 1);
  // permutation entries read as their low 32-bit words (little-endian; the
  // entries are below 2^31): a 64-bit load whose unused high word's register
  // the compiler reuses would have to be awaited before that reuse
  const int32_t* perm_lo = reinterpret_cast<const int32_t*>(g.perm);
  int prow[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int r = 8 * min(4 * q + wave, 2 * LIVE_B - 1) + (lane >> 3);
    prow[q] = row0 + min(r, rows - 1);
    if (MODE == 1) prow[q] = perm_lo[2 * (size_t)prow[q]];
  }
  const int p_d = row0 + min(drow, rows - 1);
  const int prow_d = (MODE == 0) ? p_d : perm_lo[2 * (size_t)p_d];  // mode 1: flat routed index (x row = it / topk); mode 2: output row
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int r = 8 * min(4 * q + wave, 2 * LIVE_B - 1) + (lane >> 3);
    const int src = (MODE == 1) ? prow[q] / g.topk : prow[q];
    const int c = (lane & 7) ^ (r & 7);
    // rows past the tile's last row read beyond the resource's extent, which
    // fills their LDS rows with zeros (no L2 traffic, idle multiplier
    // inputs); their results are never stored
    aoff[q] = r < rows ? 2u * ((uint32_t)src * (uint32_t)g.lda + 8u * (uint32_t)c) : 0x80000000u;
  }
  asm volatile("" ::: "memory");
  issue_chunk(live_c, 0, 0);
  if (nch > 1) issue_chunk(live_c, 1, 1);
  asm volatile("" ::: "memory");
  uint32_t mx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  {
    bool ok;
    const uint16_t* sc = se + (size_t)tile_word(tid & 31, ok) * 8;
    // up to 64 groups per round, all their loads in flight together
    // (indexes past the last group re-read it, which leaves the maxima
    // unchanged)
    for (int gb = 0; gb < G; gb += 64) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = *reinterpret_cast<const uint4*>(sc + (size_t)min(gb + (tid >> 5) + 8 * u, G - 1) * N);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          mx[2 * q] = max(mx[2 * q], vv[q] & 0x7fffu);
          mx[2 * q + 1] = max(mx[2 * q + 1], (vv[q] >> 16) & 0x7fffu);
        }
      }
    }
  }
  float row_w = 0.f;
  if (MODE == 2) row_w = bf16_to_f32(g.wts[prow_d]);
  const int row_e = g.rexp[(MODE == 1) ? prow_d / g.topk : p_d];
  asm volatile("" ::: "memory");
  // s_mx zeroed by every thread before anyone adds to it
  wait_vm_lgkm0<63>();
  barrier_no_fence();
#pragma unroll
  for (int j = 0; j < 8; ++j) lds_max4_settled(s_mx + (tid & 31) * 8 + j, mx[j]);
  // chunks 0 and 1 have landed: the loads of the maxima, issued after them
  // and already awaited, return in order; only the per-row loads (1 or 2)
  // may be pending
  constexpr int kRowLoads = (MODE == 2) ? 2 : 1;
  wait_vm_lgkm0<kRowLoads>();
  barrier_no_fence();

  // this lane's column exponents (16 * S * 2^ec has |.| in [256, 512)), in fragment order
  int ecf[4];
  {
    const u32x4_t m = lds_read16_settled(s_mx + tc_a * 8 + 4 * hi);
#pragma unroll
    for (int f = 0; f < 4; ++f) ecf[f] = exp_to(m[f], 131);
  }

  // scale pairs of the current group, per fragment: (16S', 16S') and
  // (-24S', -24S'), from the raw bf16 rows staged with the chunk (row h
  // belongs to the chunk's step h)
  uint32_t sp[4], sn[4];
  auto to_pair = [&](uint32_t b16, int f) -> uint32_t {
    const float v = ldexpf(__uint_as_float(b16 << 16), ecf[f] + 4);
    return pk_rtz(v, v);
  };
  auto load_scales = [&](int slot, int h) {
    const unsigned char* sb = lds + slot * SLOT + B_SLOT + A_SLOT + wave * 256 + h * 128;
    const u32x2_t v = lds_read8_settled(sb + (tc_a & 7) * 16 + 8 * hi);
    sp[0] = to_pair(v[0] & 0xffffu, 0);
    sp[1] = to_pair(v[0] >> 16, 1);
    sp[2] = to_pair(v[1] & 0xffffu, 2);
    sp[3] = to_pair(v[1] >> 16, 3);
#pragma unroll
    for (int f = 0; f < 4; ++f) sn[f] = times_m15(sp[f]);
  };

  const int steps_per_group = g.gs / BK;
  const uint32_t nib_mask = opaque_vreg(0x03C003C0u);
  // under the mask: the nibble with its top bit flipped (u = q + 8); elsewhere
  // fp16 exponent 15, so one v_bitop3 (0x6A: mask ? x ^ c : c) gives 1 + u/16
  const uint32_t nib_c = opaque_vreg(0x3E003E00u);
  // LDS word positions of this lane's words (k-block kb reads with swizzle 8kb)
  const int bpos_a = tc_a ^ (8 * kb);
  // v_perm selector of the nibble half this lane needs
  const uint32_t sel = (hi != 0) ? 0x07060302u : 0x05040100u;

  // one MFMA step: dequantise this lane's B fragments, then MFMA them against
  // every live row tile (LIVE is a compile-time count: no per-tile branches)
  // B words of one step for this lane: 8 k-rows of its word
  auto load_bwords = [&](int slot, int half, uint32_t (&wa)[8]) {
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(lds + slot * SLOT) + (32 * half + 8 * kb) * BWORDS;
#pragma unroll
    for (int i = 0; i < 8; ++i) wa[i] = bs[i * BWORDS + bpos_a];
  };
  auto mfma_step = [&](auto& acc, auto live_c, int slot, int half, uint32_t (&wa)[8], bool prefetch_next) {
    constexpr int LIVE = decltype(live_c)::value;
    // this lane's A fragments (16 rows x 8 k of each live row tile), read
    // before the dequantisation so their latency hides behind it
    const unsigned char* as = lds + slot * SLOT + B_SLOT + (((4 * half + kb) ^ (i16 & 7)) << 4) + i16 * 128;
    half8_t af[MT];
#pragma unroll
    for (int t = 0; t < LIVE; ++t) af[t] = *reinterpret_cast<const half8_t*>(as + t * 2048);
    uint32_t ta[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) ta[pr] = __builtin_amdgcn_perm(wa[2 * pr + 1], wa[2 * pr], sel);
    // the words of the chunk's second step land while this step computes
    if (prefetch_next) load_bwords(slot, 1, wa);
    // Dequantisation of fragment f in three stages of four independent ops
    // (nibble to position, and-or to fp16 1 + u/16, fma with the scales).
    auto dq_pos = [&](auto f_c, int pr) -> uint32_t {
      constexpr int F = decltype(f_c)::value;
      const uint32_t t = ta[pr];
      return (F == 0) ? (t << 6) : (F == 1) ? (t << 2) : (F == 2) ? (t >> 2) : (t >> 6);
    };
    auto dq_fma = [&](auto f_c, uint32_t m) -> uint32_t {
      constexpr int F = decltype(f_c)::value;
      return h2_bits(__builtin_elementwise_fma(as_h2(m), as_h2(sp[F]), as_h2(sn[F])));
    };
    uint32_t hc[4], hn[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) hn[pr] = dq_pos(IntC<0>{}, pr);
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) hn[pr] = __builtin_amdgcn_bitop3_b32(hn[pr], nib_mask, nib_c, 0x6A);
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) hc[pr] = dq_fma(IntC<0>{}, hn[pr]);
    __builtin_amdgcn_sched_barrier(0);
    // MFMAs of fragment f over the live row tiles, with the three stages of
    // fragment f+1 after the first three of them: VALU and MFMA alternate
    // within the wave, and each VALU group is independent. sched_barrier
    // keeps this order.
    auto frag = [&](auto f_c) {
      constexpr int F = decltype(f_c)::value;
      constexpr int FN = F < 3 ? F + 1 : 3;
      const half8_t bcur = __builtin_bit_cast(half8_t, make_uint4(hc[0], hc[1], hc[2], hc[3]));
#pragma unroll
      for (int t = 0; t < LIVE; ++t) {
        acc[t][F] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bcur, acc[t][F], 0, 0, 0);
        if (F < 3) {
          if (t == 0) {
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) hn[pr] = dq_pos(IntC<FN>{}, pr);
          }
          if (t == (LIVE > 1 ? 1 : 0)) {
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) hn[pr] = __builtin_amdgcn_bitop3_b32(hn[pr], nib_mask, nib_c, 0x6A);
          }
          if (t == (LIVE > 2 ? 2 : LIVE - 1)) {
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) hn[pr] = dq_fma(IntC<FN>{}, hn[pr]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) hc[pr] = hn[pr];
    };
    frag(IntC<0>{});
    frag(IntC<1>{});
    frag(IntC<2>{});
    frag(IntC<3>{});
  };

  // main loop and epilogue, specialised on the live row-tile count so that
  // only live accumulators occupy registers
  auto run = [&](auto live_c) {
    constexpr int LIVE = decltype(live_c)::value;
    f32x4_t acc[LIVE][4];
#pragma unroll
    for (int t = 0; t < LIVE; ++t)
#pragma unroll
      for (int f = 0; f < 4; ++f) acc[t][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    int gstep = 0;
    // one chunk in ring slot SLOT_C (a compile-time constant, so every LDS
    // address of the chunk is an immediate offset)
    auto chunk = [&](auto slot_c, int c) {
      constexpr int sl = decltype(slot_c)::value;
      if (c > 0) {
        // chunk c has landed once only chunk c+1 (3 + NQ DMA per thread) may be pending
        if (c + 1 < nch) wait_vm_lgkm0<3 + NQ>();
        else wait_vm_lgkm0<0>();
        barrier_no_fence();
      }
      // every wave is past chunk c-1: its ring slot takes chunk c+2
      if (c + 2 < nch) issue_chunk(live_c, c + 2, (sl + NC - 1) % NC);
      uint32_t wa[8];
      load_bwords(sl, 0, wa);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        if (gstep == 0) load_scales(sl, half);
        mfma_step(acc, live_c, sl, half, wa, half == 0);
        if (++gstep == steps_per_group) gstep = 0;
      }
    };
    static_assert(NC == 3, "the main loop is unrolled over the three ring slots");
    for (int c = 0; c < nch; c += NC) {
      chunk(IntC<0>{}, c);
      if (c + 1 < nch) chunk(IntC<1>{}, c + 1);
      if (c + 2 < nch) chunk(IntC<2>{}, c + 2);
    }
  // ---- per-row data to LDS for the epilogue
  if (tid < BM) {
    s_erow[tid] = drow < rows ? row_e : 0;
    if (MODE == 2) {
      s_orow[tid] = prow_d;
      s_wrow[tid] = row_w;
    }
    if (MODE == 1) s_rmax[tid] = 0u;
  }
  __syncthreads();

  // ---- epilogue. MFMA 16x16 layout: lane holds column i16 of fragment f
  // for rows 4*kb + r, r = 0..3, of each row tile.
#pragma unroll
  for (int t = 0; t < LIVE; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * t + 4 * kb + r;
      const bool ok = row < rows && col_ok;
      const int er = s_erow[row];
      float v[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) v[f] = ldexpf(acc[t][f][r], -(er + ecf[f]));
      if (MODE == 1) {
        // gate lanes ((i16 & 4) == 0) take the up values of act columns
        // outcol..outcol+3 from lane i16 + 4 (DPP row_shl:4)
        float u[4];
#pragma unroll
        for (int f = 0; f < 4; ++f)
          u[f] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[f]), 0x104, 0xf, 0xf, false));
        const uint32_t g01 = pk_bf16(v[0], v[1]), g23 = pk_bf16(v[2], v[3]);
        const uint32_t u01 = pk_bf16(u[0], u[1]), u23 = pk_bf16(u[2], u[3]);
        const uint32_t a01 = pk_bf16(silu_f32(bf16_lo(g01)) * bf16_lo(u01), silu_f32(bf16_hi(g01)) * bf16_hi(u01));
        const uint32_t a23 = pk_bf16(silu_f32(bf16_lo(g23)) * bf16_lo(u23), silu_f32(bf16_hi(g23)) * bf16_hi(u23));
        const bool gate_ok = ok && (i16 & 4) == 0;
        if (gate_ok) *reinterpret_cast<uint2*>(g.y + (size_t)(row0 + row) * g.ldy + outcol) = make_uint2(a01, a23);
        const uint32_t amax = row16_max(gate_ok ? max(max(a01 & 0x7fffu, (a01 >> 16) & 0x7fffu),
                                                      max(a23 & 0x7fffu, (a23 >> 16) & 0x7fffu))
                                                : 0u);
        if (i16 == 0) atomicMax(s_rmax + row, amax);
      } else if (MODE == 2) {
        if (ok) {
          const float wv = s_wrow[row];
          const uint32_t p01 = pk_bf16(v[0], v[1]), p23 = pk_bf16(v[2], v[3]);
          *reinterpret_cast<uint2*>(g.y + (size_t)s_orow[row] * g.ldy + outcol) =
              make_uint2(pk_bf16(bf16_lo(p01) * wv, bf16_hi(p01) * wv), pk_bf16(bf16_lo(p23) * wv, bf16_hi(p23) * wv));
        }
      } else {
        if (ok)
          *reinterpret_cast<uint2*>(g.y + (size_t)(row0 + row) * g.ldy + outcol) =
              make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]));
      }
    }
  }
  if (MODE == 1) {
    __syncthreads();
    if (tid < rows && s_rmax[tid] != 0u) atomicMax(g.rmax_out + row0 + tid, s_rmax[tid]);
  }
  };
  run(live_c);
  };
  switch (live) {
    case 1: body(IntC<1>{}); break;
    case 2: body(IntC<2>{}); break;
    case 3: body(IntC<3>{}); break;
    case 4: body(IntC<4>{}); break;
    case 5: body(IntC<5>{}); break;
    case 6: body(IntC<6>{}); break;
    case 7: body(IntC<7>{}); break;
    default: body(IntC<8>{}); break;
  }


}

// Per-row exponent and fp16 copy of bf16 rows: e = exponent that puts
// max |x| * 2^e in [2^13, 2^14), x16 = fp16(x * 2^e) (exact: a bf16 value
// keeps its 8 significant bits; values below 2^-30 of the row maximum, which
// fp16's subnormals cannot hold exactly, round toward zero). One wave per
// row; rows of up to 4096 columns are read once into registers (all loads in
// flight together), longer ones in two passes. `rmax` (optional) gives the
// row maxima instead of a scan. Also clears an optional buffer of `nzero`
// words.
constexpr int kRowRegs = 8;  // 16-byte pieces per lane held in registers
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
  _Float16* yr = x16 + (size_t)row * K;
  auto convert = [&](const uint4& v, float sc, int c) {
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      h[q] = pk_rtz(__uint_as_float(vv[q] << 16) * sc, __uint_as_float(vv[q] & 0xffff0000u) * sc);
    *reinterpret_cast<uint4*>(yr + c) = make_uint4(h[0], h[1], h[2], h[3]);
  };
  auto vmax = [](uint32_t m, const uint4& v) {
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) m = max(m, max(vv[q] & 0x7fffu, (vv[q] >> 16) & 0x7fffu));
    return m;
  };
  if (K <= kRowRegs * 512) {
    uint4 v[kRowRegs];
#pragma unroll
    for (int i = 0; i < kRowRegs; ++i) {
      const int c = lane * 8 + 512 * i;
      v[i] = c < K ? *reinterpret_cast<const uint4*>(xr + c) : make_uint4(0u, 0u, 0u, 0u);
    }
    uint32_t m;
    if (rmax != nullptr) {
      m = rmax[row];
    } else {
      m = 0;
#pragma unroll
      for (int i = 0; i < kRowRegs; ++i) m = vmax(m, v[i]);
      m = wave_max_u32(m);
    }
    const int e = exp_to(m, 140);
    if (lane == 0) rexp[row] = e;
    const float sc = ldexpf(1.0f, e);
#pragma unroll
    for (int i = 0; i < kRowRegs; ++i) {
      const int c = lane * 8 + 512 * i;
      if (c < K) convert(v[i], sc, c);
    }
    return;
  }
  uint32_t m = 0;
  if (rmax != nullptr) {
    m = rmax[row];
  } else {
    for (int c = lane * 8; c < K; c += 512) m = vmax(m, *reinterpret_cast<const uint4*>(xr + c));
    m = wave_max_u32(m);
  }
  const int e = exp_to(m, 140);
  if (lane == 0) rexp[row] = e;
  const float sc = ldexpf(1.0f, e);
  for (int c = lane * 8; c < K; c += 512) convert(*reinterpret_cast<const uint4*>(xr + c), sc, c);
}

// out[t, n] = bf16(sum_{j < k, in order} prod[t*k + j, n]) (+ shared, a bf16 add)
__global__ __launch_bounds__(1024) void slot_reduce_kernel(const uint16_t* __restrict__ prod, int T, int k, int H,
                                                          const uint16_t* __restrict__ shared,
                                                          uint16_t* __restrict__ out) {
  const int c8 = blockIdx.x * blockDim.x + threadIdx.x;  // group of 8 columns
  if (8 * c8 >= H) return;
  for (int t = blockIdx.y; t < T; t += gridDim.y) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    // the k product rows of the token in flight together, summed in slot order
    // (nontemporal: every product is read once)
    u32x4_t pv[QMOE_KMAX];
#pragma unroll
    for (int j = 0; j < QMOE_KMAX; ++j)
      if (j < k) pv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(prod + ((size_t)t * k + j) * H + 8 * c8));
#pragma unroll
    for (int j = 0; j < QMOE_KMAX; ++j) {
      if (j < k) {
        const uint32_t vv[4] = {pv[j][0], pv[j][1], pv[j][2], pv[j][3]};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a[2 * q] += bf16_to_f32(vv[q] & 0xffffu);
          a[2 * q + 1] += bf16_to_f32(vv[q] >> 16);
        }
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

constexpr size_t kGemmLds = (size_t)NC * SLOT + 256 * sizeof(uint32_t) + 4 * BM * sizeof(int);
static_assert(kGemmLds <= 80 * 1024, "two workgroups per CU");

template <int MODE>
int launch_gemm(const GemmArgs& a, int mtiles_max, hipStream_t st) {
  // grid: every XCD gets ceil(row tiles / 8) row tiles with all their column tiles
  const long nblk = 8L * ((mtiles_max + 7) / 8) * a.n_ntiles;
  if (nblk <= 0) return 0;
  if (nblk > 0x7fffffffL) return QMOE_EINVAL;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  static bool attr_set[64] = {};
  if (dev < 0 || dev >= 64) return QMOE_EINVAL;
  if (!attr_set[dev]) {
    err = hipFuncSetAttribute((const void*)grouped_gemm_f16_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kGemmLds);
    if (err != hipSuccess) return (int)err;
    attr_set[dev] = true;
  }
  GemmArgs b = a;
  b.mtiles_max = mtiles_max;
  hipLaunchKernelGGL((grouped_gemm_f16_kernel<MODE>), dim3((unsigned)nblk), dim3(kThreads),
                     kGemmLds, st, b);
  return (int)hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// tensors the GEMM reads through buffer resources (activations, one expert's
// weights) must fit their 31-bit extent
bool buffer_extent_ok(size_t bytes) { return bytes > 0 && bytes < 0x80000000ull; }

int launch_rows_to_f16(const void* x, int rows, int K, const uint32_t* rmax, int* rexp, _Float16* x16,
                       uint32_t* zero, int nzero, hipStream_t st) {
  const int blocks = max(host_ceil_div(rows, 4), host_ceil_div(nzero, 256));
  hipLaunchKernelGGL(rows_to_f16_kernel, dim3(max(blocks, 1)), dim3(256), 0, st, (const uint16_t*)x, rows, K, rmax,
                     rexp, x16, zero, nzero);
  return (int)hipGetLastError();
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

bool gemm_shape_ok(int K, int N, int gs) {
  return K >= KC && K % KC == 0 && N >= 32 && N % 32 == 0 && gs >= BK && gs % BK == 0 && K % gs == 0;
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
  if (!buffer_extent_ok((size_t)R * K * 2) || !buffer_extent_ok((size_t)K * N / 2)) return QMOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  _Float16* x16 = (_Float16*)workspace;
  int* rexp = (int*)((char*)workspace + align256((size_t)R * K * 2));
  int rc = launch_rows_to_f16(x, R, K, nullptr, rexp, x16, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a16 = x16; a.lda = K; a.a_bytes = (uint32_t)((size_t)R * K * 2); a.perm = nullptr; a.topk = 1; a.rexp = rexp;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(N, 256); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, mtiles_max, st);
}

size_t qmoe_w4a16_gemm_mfma_workspace(int M, int K) { return plain_ws(M > 0 ? M : 1, K); }

int qmoe_w4a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int gs,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 1 || !gemm_shape_ok(K, N, gs) || !aligned16(x) || !aligned16(y) || !aligned16(scale) ||
      !aligned16(workspace))
    return QMOE_EINVAL;
  if (workspace_bytes < qmoe_w4a16_gemm_mfma_workspace(M, K)) return QMOE_EWORKSPACE;
  if (!buffer_extent_ok((size_t)M * K * 2) || !buffer_extent_ok((size_t)K * N / 2)) return QMOE_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  _Float16* x16 = (_Float16*)workspace;
  int* rexp = (int*)((char*)workspace + align256((size_t)M * K * 2));
  int rc = launch_rows_to_f16(x, M, K, nullptr, rexp, x16, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a16 = x16; a.lda = K; a.a_bytes = (uint32_t)((size_t)M * K * 2); a.topk = 1; a.rexp = rexp;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.R = M; a.n_ntiles = host_ceil_div(N, 256); a.y = (uint16_t*)y; a.ldy = N;
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
  if (T < 1 || k < 1 || k > QMOE_KMAX || E < 1 || !gemm_shape_ok(H, 2 * MI, gs_gu) || !gemm_shape_ok(MI, H, gs_dn) ||
      !aligned16(x) || !aligned16(out) || !aligned16(gu_s) || !aligned16(dn_s) || !aligned16(workspace) ||
      (shared != nullptr && !aligned16(shared)) || tile_expert == nullptr)
    return QMOE_EINVAL;
  const PrefillLayout l = prefill_layout(T, k, H, MI);
  if (workspace_bytes < l.total) return QMOE_EWORKSPACE;
  if (!buffer_extent_ok((size_t)T * H * 2) || !buffer_extent_ok((size_t)T * k * MI * 2) ||
      !buffer_extent_ok((size_t)H * MI))
    return QMOE_EINVAL;
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
  a.a16 = x16; a.lda = H; a.a_bytes = (uint32_t)((size_t)T * H * 2); a.perm = (const int64_t*)order; a.topk = k; a.rexp = rexp_x; a.rmax_out = rmax;
  a.w = (const uint32_t*)gu_w; a.s = (const uint16_t*)gu_s; a.K = H; a.N = 2 * MI; a.gs = gs_gu;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(MI, 128); a.y = act; a.ldy = MI; a.MI = MI;
  rc = launch_gemm<1>(a, mtiles_max, st);
  if (rc) return rc;
  rc = launch_rows_to_f16(act, R, MI, rmax, rexp_a, act16, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs d = a;
  d.a16 = act16; d.lda = MI; d.a_bytes = (uint32_t)((size_t)R * MI * 2); d.perm = (const int64_t*)order; d.topk = k; d.rexp = rexp_a; d.rmax_out = nullptr;
  d.w = (const uint32_t*)dn_w; d.s = (const uint16_t*)dn_s; d.K = MI; d.N = H; d.gs = gs_dn;
  d.n_ntiles = host_ceil_div(H, 256); d.y = prod; d.ldy = H; d.wts = (const uint16_t*)wts;
  rc = launch_gemm<2>(d, mtiles_max, st);
  if (rc) return rc;
  // one workgroup row covers a token's H / 8 column groups (whole waves, at most 1024 threads), so no
  // thread of a launched block idles when H / 8 is a multiple of 64
  const int sr_threads = min(1024, host_ceil_div(H / 8, 64) * 64);
  hipLaunchKernelGGL(slot_reduce_kernel, dim3(host_ceil_div(H / 8, sr_threads), min(T, 65535)), dim3(sr_threads), 0, st, prod, T,
                     k, H, (const uint16_t*)shared, (uint16_t*)out);
  return (int)hipGetLastError();
}

}  // extern "C"
