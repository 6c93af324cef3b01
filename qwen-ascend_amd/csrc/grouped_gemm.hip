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
constexpr int LDA = KC + 8;      // fp16 per staged A row (16-byte padding)
constexpr int WAVE_COLS = 128;   // output columns per wave (16 word-columns)

struct GemmArgs {
  const uint16_t* a;         // bf16 activations, row stride lda
  int lda;
  const int64_t* perm;       // mode 1: a row of p = perm[p] / topk; mode 2: output row of p = perm[p]
  int topk;
  const int* rexp;           // per a-row exponent (indexed like the a row), or nullptr: from rmax_in
  const uint32_t* rmax_in;   // per permuted row max |a| (bf16 bits), used when rexp is nullptr
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
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDA];
  __shared__ int s_erow[BM];

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

  // ---- this lane's word-column (8 output columns)
  int wcol;
  bool col_ok;
  int outcol0;  // first output column of the word (mode 1: act column)
  if (MODE == 1) {
    const int a0 = nt * 256 + 8 * (8 * wave + (i16 & 7));  // act column of the word
    col_ok = a0 < g.MI;
    outcol0 = a0;
    wcol = ((i16 < 8) ? a0 : g.MI + a0) >> 3;
  } else {
    outcol0 = nt * 512 + wave * WAVE_COLS + 8 * i16;
    col_ok = outcol0 < N;
    wcol = outcol0 >> 3;
  }
  if (!col_ok) wcol = 0;  // keep loads in bounds; results are not stored

  const uint32_t* we = g.w + (size_t)e * K * nw + wcol;
  const uint16_t* se = g.s + (size_t)e * G * N + (size_t)wcol * 8;

  // ---- column exponents: max over all groups of |S| of the word's 8 columns
  int ec[8];
  {
    uint32_t mx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int gi = 0; gi < G; ++gi) {
      const uint4 v = *reinterpret_cast<const uint4*>(se + (size_t)gi * N);
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

  // ---- A staging: thread -> (row r = tid/2, 32 k of the 64-k chunk)
  const int ar = tid >> 1, ah = tid & 1;
  const bool arow_ok = ar < rows;
  const uint16_t* asrc;
  int aexp = 0;
  {
    const int p = row0 + min(ar, rows - 1);
    int src = p;
    if (MODE == 1 && g.perm != nullptr) src = (int)(g.perm[p] / g.topk);
    asrc = g.a + (size_t)src * g.lda + 32 * ah;
    if (g.rexp != nullptr) aexp = g.rexp[src];
    else aexp = exp_to(g.rmax_in[p], 140);
    if (ah == 0) s_erow[ar] = arow_ok ? aexp : 0;
  }
  const float ascale = ldexpf(1.0f, aexp);
  uint4 areg[4];
  auto load_a = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      areg[q] = arow_ok ? *reinterpret_cast<const uint4*>(asrc + k0 + 8 * q) : make_uint4(0, 0, 0, 0);
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t v[4] = {areg[q].x, areg[q].y, areg[q].z, areg[q].w};
      uint32_t h[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        h[c] = pk_rtz(__uint_as_float(v[c] << 16) * ascale, __uint_as_float(v[c] & 0xffff0000u) * ascale);
      *reinterpret_cast<uint4*>(&As[buf][ar * LDA + 32 * ah + 8 * q]) = make_uint4(h[0], h[1], h[2], h[3]);
    }
  };

  // ---- B: 8 words (rows k0 + 8kb + i of the word-column) per MFMA step
  auto load_b = [&](uint32_t (&dst)[8], int k0) {
    const uint32_t* p = we + (size_t)(k0 + 8 * kb) * nw;
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = p[(size_t)i * nw];
  };

  // scale pairs of the current group for the word's 8 columns: (16S', 16S') and (-24S', -24S')
  uint32_t sp[8], sn[8];
  auto load_scales = [&](int grp) {
    const uint4 v = *reinterpret_cast<const uint4*>(se + (size_t)grp * N);
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

  const int nsteps = K / BK;  // even: K is a multiple of KC = 2 * BK
  const int steps_per_group = g.gs / BK;

  // one MFMA step: dequantise the 8x8 nibble block held in w[] into 8 fp16
  // B fragments, then MFMA them against every live row tile
  auto mfma_step = [&](const uint32_t (&w)[8], int buf, int half) {
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
    const int kofs = half * BK + 8 * kb;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < live) {
        const half8_t af = *reinterpret_cast<const half8_t*>(&As[buf][(16 * t + i16) * LDA + kofs]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[t][j], 0, 0, 0);
      }
    }
  };

  // prologue: A chunk 0 staged, B of steps 0 and 1 in flight
  uint32_t b0[8], b1[8];
  load_a(0);
  store_a(0);
  load_b(b0, 0);
  load_b(b1, BK);
  __syncthreads();

  // one iteration = one 64-k chunk = two MFMA steps; B of the next chunk is
  // loaded while this chunk computes
  for (int c = 0; c < nsteps / 2; ++c) {
    const int buf = c & 1;
    const bool more = (c + 1) * KC < K;
    if (more) load_a((c + 1) * KC);
    uint32_t w0[8], w1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { w0[i] = b0[i]; w1[i] = b1[i]; }
    if (more) {
      load_b(b0, (c + 1) * KC);
      load_b(b1, (c + 1) * KC + BK);
    }
    if ((2 * c) % steps_per_group == 0) load_scales((2 * c) / steps_per_group);
    mfma_step(w0, buf, 0);
    if ((2 * c + 1) % steps_per_group == 0) load_scales((2 * c + 1) / steps_per_group);
    mfma_step(w1, buf, 1);
    if (more) store_a(buf ^ 1);
    __syncthreads();
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

// Per-row exponent of bf16 rows (max |x| * 2^e in [2^13, 2^14)), one wave
// per row; also clears an optional buffer of `nzero` words.
__global__ __launch_bounds__(256) void row_exponent_kernel(const uint16_t* __restrict__ x, int rows, int K,
                                                           int* __restrict__ rexp, uint32_t* __restrict__ zero,
                                                           int nzero) {
  const int gtid = blockIdx.x * 256 + threadIdx.x;
  for (int q = gtid; q < nzero; q += gridDim.x * 256) zero[q] = 0u;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* xr = x + (size_t)row * K;
  uint32_t m = 0;
  for (int c = lane * 8; c < K; c += 512) {
    const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) m = max(m, max(vv[q] & 0x7fffu, (vv[q] >> 16) & 0x7fffu));
  }
  m = wave_max_u32(m);
  if (lane == 0) rexp[row] = exp_to(m, 140);
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

template <int MODE>
int launch_gemm(const GemmArgs& a, int mtiles_max, hipStream_t st) {
  const long nblk = (long)mtiles_max * a.n_ntiles;
  if (nblk <= 0) return 0;
  hipLaunchKernelGGL((grouped_gemm_f16_kernel<MODE>), dim3((unsigned)nblk), dim3(kThreads), 0, st, a);
  return (int)hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launch_row_exponent(const void* x, int rows, int K, int* rexp, uint32_t* zero, int nzero, hipStream_t st) {
  const int blocks = max(host_ceil_div(rows, 4), host_ceil_div(nzero, 256));
  hipLaunchKernelGGL(row_exponent_kernel, dim3(max(blocks, 1)), dim3(256), 0, st, (const uint16_t*)x, rows, K, rexp,
                     zero, nzero);
  return (int)hipGetLastError();
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// workspace of the fused prefill: act [R, MI] bf16 | prod [R, H] bf16 | x row exponents [T] | act row max [R]
void prefill_layout(int T, int k, int H, int MI, size_t* o_prod, size_t* o_rexp, size_t* o_rmax, size_t* total) {
  const size_t R = (size_t)T * k;
  size_t o = align256(R * MI * 2);
  *o_prod = o;
  o += align256(R * H * 2);
  *o_rexp = o;
  o += align256((size_t)T * 4);
  *o_rmax = o;
  o += align256(R * 4);
  *total = o;
}

}  // namespace

// ============================================================================ C ABI

extern "C" {

int qmoe_gemm_tile_rows(void) { return BM; }

size_t qmoe_grouped_gemm_workspace(int R) { return align256((size_t)(R > 0 ? R : 1) * sizeof(int)); }

int qmoe_grouped_gemm(const void* x, int R, int K, int N, int E, int gs, const void* w, const void* scale,
                      const void* tile_expert, const void* tile_row0, const void* tile_rows,
                      const void* tile_count, int mtiles_max, void* y, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (R < 0 || K < KC || (K % KC) || N < 8 || (N % 8) || E < 1 || gs < BK || (gs % BK) || (K % gs) ||
      !aligned16(x) || !aligned16(y) || !aligned16(scale) || tile_expert == nullptr)
    return QMOE_EINVAL;
  if (R == 0) return 0;
  if (workspace_bytes < qmoe_grouped_gemm_workspace(R)) return QMOE_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  int* rexp = (int*)workspace;
  int rc = launch_row_exponent(x, R, K, rexp, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a = (const uint16_t*)x; a.lda = K; a.perm = nullptr; a.topk = 1; a.rexp = rexp;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(N, 512); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, mtiles_max, st);
}

size_t qmoe_w4a16_gemm_mfma_workspace(int M) { return align256((size_t)(M > 0 ? M : 1) * sizeof(int)); }

int qmoe_w4a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int gs,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 1 || K < KC || (K % KC) || N < 8 || (N % 8) || gs < BK || (gs % BK) || (K % gs) || !aligned16(x) ||
      !aligned16(y) || !aligned16(scale))
    return QMOE_EINVAL;
  if (workspace_bytes < qmoe_w4a16_gemm_mfma_workspace(M)) return QMOE_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  int* rexp = (int*)workspace;
  int rc = launch_row_exponent(x, M, K, rexp, nullptr, 0, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a = (const uint16_t*)x; a.lda = K; a.topk = 1; a.rexp = rexp;
  a.w = (const uint32_t*)w; a.s = (const uint16_t*)scale; a.K = K; a.N = N; a.gs = gs;
  a.R = M; a.n_ntiles = host_ceil_div(N, 512); a.y = (uint16_t*)y; a.ldy = N;
  return launch_gemm<0>(a, host_ceil_div(M, BM), st);
}

size_t qmoe_moe_prefill_workspace(int T, int k, int H, int MI) {
  size_t a, b, c, total;
  prefill_layout(T, k, H, MI, &a, &b, &c, &total);
  return total;
}

int qmoe_moe_experts_grouped(const void* x, int T, int H, int MI, int E, int k, const void* wts,
                             const void* order, const void* gu_w, const void* gu_s, int gs_gu,
                             const void* dn_w, const void* dn_s, int gs_dn, const void* tile_expert,
                             const void* tile_row0, const void* tile_rows, const void* tile_count,
                             int mtiles_max, const void* shared, void* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (T < 1 || k < 1 || E < 1 || H < KC || (H % KC) || MI < KC || (MI % KC) || gs_gu < BK || (gs_gu % BK) ||
      (H % gs_gu) || gs_dn < BK || (gs_dn % BK) || (MI % gs_dn) || !aligned16(x) || !aligned16(out) ||
      !aligned16(gu_s) || !aligned16(dn_s) || (shared != nullptr && !aligned16(shared)) || tile_expert == nullptr)
    return QMOE_EINVAL;
  size_t o_prod, o_rexp, o_rmax, total;
  prefill_layout(T, k, H, MI, &o_prod, &o_rexp, &o_rmax, &total);
  if (workspace_bytes < total) return QMOE_EWORKSPACE;
  const int R = T * k;
  char* ws = (char*)workspace;
  uint16_t* act = (uint16_t*)ws;
  uint16_t* prod = (uint16_t*)(ws + o_prod);
  int* rexp = (int*)(ws + o_rexp);
  uint32_t* rmax = (uint32_t*)(ws + o_rmax);
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_row_exponent(x, T, H, rexp, rmax, R, st);
  if (rc) return rc;
  GemmArgs a{};
  a.a = (const uint16_t*)x; a.lda = H; a.perm = (const int64_t*)order; a.topk = k; a.rexp = rexp;
  a.rmax_out = rmax;
  a.w = (const uint32_t*)gu_w; a.s = (const uint16_t*)gu_s; a.K = H; a.N = 2 * MI; a.gs = gs_gu;
  a.tile_expert = (const int*)tile_expert; a.tile_row0 = (const int*)tile_row0;
  a.tile_rows = (const int*)tile_rows; a.tile_count = (const int*)tile_count; a.R = R;
  a.n_ntiles = host_ceil_div(MI, 256); a.y = act; a.ldy = MI; a.MI = MI;
  rc = launch_gemm<1>(a, mtiles_max, st);
  if (rc) return rc;
  GemmArgs d = a;
  d.a = act; d.lda = MI; d.perm = (const int64_t*)order; d.topk = k; d.rexp = nullptr; d.rmax_in = rmax;
  d.rmax_out = nullptr;
  d.w = (const uint32_t*)dn_w; d.s = (const uint16_t*)dn_s; d.K = MI; d.N = H; d.gs = gs_dn;
  d.n_ntiles = host_ceil_div(H, 512); d.y = prod; d.ldy = H; d.wts = (const uint16_t*)wts;
  rc = launch_gemm<2>(d, mtiles_max, st);
  if (rc) return rc;
  hipLaunchKernelGGL(slot_reduce_kernel, dim3(host_ceil_div(H / 8, 256), min(T, 65535)), dim3(256), 0, st, prod, T,
                     k, H, (const uint16_t*)shared, (uint16_t*)out);
  return (int)hipGetLastError();
}

}  // extern "C"
