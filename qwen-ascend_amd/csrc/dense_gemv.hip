// Dense bf16 projections around the expert block: the shared expert and the
// router (fnx/engine.py:1786-1802), as one to four token rows.
//
//   y[m, n] = bf16( sum_k a[m, k] * W[n, k] )   (F.linear, fp32 accumulation)
//
// W is a bf16 [N, K] row-major matrix (the reference's Raw container), so
// every output is a dot product over one contiguous weight row. A wave owns
// RPW rows; lane l takes the 16-byte pieces l, l+64, ... of each row (8 bf16
// each), so a wave's loads of one row are fully coalesced, and all RPW rows
// are in flight before the first dot product. Per row, the lane's partial
// (v_dot2_f32_bf16 over its pieces, in piece order) is summed over the wave
// by DPP in a fixed tree: results are deterministic run to run.
//
// Output columns n >= split go to a second matrix y2 (column n - split): the
// fused shared/router projection hands the router logits to the decode
// kernels as their own 16-byte aligned rows.
//
// Activations a: x itself (mode 0), or the shared expert's SwiGLU computed
// from the first projection's output gu (mode 1):
//   a[m, k] = bf16( bf16(silu(g)) * u ),  g = gu[m, k], u = gu[m, MI + k]
// the bf16 arithmetic of F.silu(gu[:, :MI]) * gu[:, MI:2MI]
// (fnx/engine.py:1788).
#include "qmoe_common.h"
#include "qmoe.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxM = 4;

QMOE_DEV bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// bf16(bf16(silu(g)) * u) for one element, both operands bf16 bits.
QMOE_DEV uint32_t swiglu_bf16_elem(uint32_t g, uint32_t u) { return swiglu_bf16_bits(g, u); }

// Activation piece i (8 bf16 at k = 8*(lane + 64 i)) of row m, as 4 words.
template <int MODE>
QMOE_DEV uint4 act_piece(const uint16_t* __restrict__ a, long lda, int m, int k, int K, int MI) {
  if (k >= K) return make_uint4(0u, 0u, 0u, 0u);
  if constexpr (MODE == 0) {
    return *reinterpret_cast<const uint4*>(a + m * lda + k);
  } else {
    const uint4 g = *reinterpret_cast<const uint4*>(a + m * lda + k);
    const uint4 u = *reinterpret_cast<const uint4*>(a + m * lda + MI + k);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = swiglu_bf16_elem(gw[q] & 0xffffu, uw[q] & 0xffffu) | (swiglu_bf16_elem(gw[q] >> 16, uw[q] >> 16) << 16);
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <int MR, int PPL, int RPW, int MODE>
__global__ __launch_bounds__(kThreads) void bf16_gemv_kernel(const uint16_t* __restrict__ a, long lda,
                                                             const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                             long ldy, uint16_t* __restrict__ y2, long ldy2, int split,
                                                             int M, int K, int N, int MI) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * kWaves + wave) * RPW;
  if (n0 >= N) return;  // whole wave
  // weights of the wave's rows first (all in flight), then the activations
  uint4 wv[RPW][PPL];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int k = 8 * (lane + 64 * i);
      wv[r][i] = (n0 + r < N && k < K) ? *reinterpret_cast<const uint4*>(w + (size_t)(n0 + r) * K + k)
                                       : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  uint4 av[MR][PPL];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int i = 0; i < PPL; ++i)
      av[m][i] = (m < M) ? act_piece<MODE>(a, lda, m, 8 * (lane + 64 * i), K, MI) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      acc[m] = 0.f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        const uint4 wq = wv[r][i], aq = av[m][i];
        acc[m] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wq.x), as_bf16x2(aq.x), acc[m], false);
        acc[m] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wq.y), as_bf16x2(aq.y), acc[m], false);
        acc[m] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wq.z), as_bf16x2(aq.z), acc[m], false);
        acc[m] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wq.w), as_bf16x2(aq.w), acc[m], false);
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float s = wave_sum_f32(acc[m]);
      const int n = n0 + r;
      if (lane == 0 && m < M && n < N) {
        uint16_t* dst = (n < split) ? y + m * ldy + n : y2 + m * ldy2 + (n - split);
        *dst = (uint16_t)f32_to_bf16(s);
      }
    }
  }
}

// act[r, i] = bf16(bf16(silu(g)) * u), g = gu[r, i], u = gu[r, MI + i] (row stride ldgu).
__global__ __launch_bounds__(kThreads) void swiglu_bf16_kernel(const uint16_t* __restrict__ gu, long ldgu,
                                                               uint16_t* __restrict__ act, long rows, int MI) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= MI) return;
  for (long r = blockIdx.y; r < rows; r += gridDim.y)
    act[r * MI + i] = (uint16_t)swiglu_bf16_elem(gu[r * ldgu + i], gu[r * ldgu + MI + i]);
}

// out[r, c] = bf16( bf16(sigmoid(gate[r])) * sh[r, c] ): torch.sigmoid(gate) * sh
// on bf16 tensors (fnx/engine.py:1793); gate element r at gate[r * ldg].
__global__ __launch_bounds__(kThreads) void shared_gate_kernel(const uint16_t* __restrict__ sh,
                                                               const uint16_t* __restrict__ gate, long ldg,
                                                               uint16_t* __restrict__ out, long rows, int H) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= H) return;
  for (long r = blockIdx.y; r < rows; r += gridDim.y) {
    const float g = bf16_to_f32(gate[r * ldg]);
    const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
    out[r * H + c] = (uint16_t)f32_to_bf16(sg * bf16_to_f32(sh[r * H + c]));
  }
}

// The same, eight columns per thread (16-byte loads and stores) when rows are
// whole 16-byte pieces: H % 8 == 0 and sh, out 16-byte aligned.
__global__ __launch_bounds__(kThreads) void shared_gate_vec_kernel(const uint16_t* __restrict__ sh,
                                                                   const uint16_t* __restrict__ gate, long ldg,
                                                                   uint16_t* __restrict__ out, long rows, int H) {
  const int c8 = blockIdx.x * kThreads + threadIdx.x;  // group of 8 columns
  if (8 * c8 >= H) return;
  for (long r = blockIdx.y; r < rows; r += gridDim.y) {
    const float g = bf16_to_f32(gate[r * ldg]);
    const float sg = round_bf16(1.0f / (1.0f + expf(-g)));
    const uint4 v = *reinterpret_cast<const uint4*>(sh + r * H + 8 * c8);
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = f32_to_bf16(sg * bf16_to_f32(in[q] & 0xffffu)) | (f32_to_bf16(sg * bf16_to_f32(in[q] >> 16)) << 16);
    *reinterpret_cast<uint4*>(out + r * H + 8 * c8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Rows per wave: as many as keep PPL * RPW <= 8 loads in flight per lane,
// but few enough that the launch has >= 256 workgroups (one CU streams only a
// small share of HBM bandwidth, so a thin grid cannot reach it).
static int pick_rpw(int ppl, int N) {
  int rpw = 8 / ppl;
  while (rpw > 1 && host_ceil_div(N, kWaves * rpw) < 256) rpw >>= 1;
  return rpw < 1 ? 1 : rpw;
}

template <int MODE>
int launch_gemv(const void* a, long lda, const void* w, void* y, long ldy, void* y2, long ldy2, int split, int M,
                int K, int N, int MI, hipStream_t st) {
  const int pieces = host_ceil_div(K, 8);
  const int ppl = pieces <= 64 ? 1 : pieces <= 128 ? 2 : pieces <= 256 ? 4 : 8;
  const int rpw = pick_rpw(ppl, N);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(host_ceil_div(N, kWaves * rpw)), dim3(kThreads), 0, st, (const uint16_t*)a, lda,
                       (const uint16_t*)w, (uint16_t*)y, ldy, (uint16_t*)y2, ldy2, split, M, K, N, MI);
    return (int)hipGetLastError();
  };
#define QMOE_GEMV_M(PPL_, RPW_)                                              \
  if (ppl == PPL_ && rpw == RPW_) {                                          \
    if (M == 1) return go(bf16_gemv_kernel<1, PPL_, RPW_, MODE>);            \
    if (M == 2) return go(bf16_gemv_kernel<2, PPL_, RPW_, MODE>);            \
    return go(bf16_gemv_kernel<4, PPL_, RPW_, MODE>);                        \
  }
  QMOE_GEMV_M(1, 8) QMOE_GEMV_M(1, 4) QMOE_GEMV_M(1, 2) QMOE_GEMV_M(1, 1)
  QMOE_GEMV_M(2, 4) QMOE_GEMV_M(2, 2) QMOE_GEMV_M(2, 1)
  QMOE_GEMV_M(4, 2) QMOE_GEMV_M(4, 1)
  QMOE_GEMV_M(8, 1)
#undef QMOE_GEMV_M
  return QMOE_EINVAL;
}

}  // namespace

extern "C" {

int qmoe_bf16_gemv(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N, void* stream) {
  if (M < 1 || M > kMaxM || K < 8 || (K % 8) || K > 8 * 64 * 8 || N < 1 || ldx < K || ldy < N || (ldx % 8))
    return QMOE_EINVAL;
  return launch_gemv<0>(x, ldx, w, y, ldy, nullptr, 0, N, M, K, N, 0, (hipStream_t)stream);
}

int qmoe_bf16_gemv_split(const void* x, long ldx, const void* w, void* y, long ldy, void* y2, long ldy2, int split,
                         int M, int K, int N, void* stream) {
  if (M < 1 || M > kMaxM || K < 8 || (K % 8) || K > 8 * 64 * 8 || N < 1 || ldx < K || (ldx % 8) || split < 0 ||
      split > N || ldy < split || (split < N && (y2 == nullptr || ldy2 < N - split)))
    return QMOE_EINVAL;
  return launch_gemv<0>(x, ldx, w, y, ldy, y2, ldy2, split, M, K, N, 0, (hipStream_t)stream);
}

int qmoe_bf16_gemv_swiglu(const void* gu, long ldgu, const void* w, void* y, long ldy, int M, int MI, int N,
                          void* stream) {
  if (M < 1 || M > kMaxM || MI < 8 || (MI % 8) || MI > 8 * 64 * 8 || N < 1 || ldgu < 2 * MI || ldy < N ||
      (ldgu % 8))
    return QMOE_EINVAL;
  return launch_gemv<1>(gu, ldgu, w, y, ldy, nullptr, 0, N, M, MI, N, MI, (hipStream_t)stream);
}

int qmoe_swiglu_bf16(const void* gu, long ldgu, void* act, long rows, int MI, void* stream) {
  if (rows < 0 || MI < 1 || ldgu < 2 * MI) return QMOE_EINVAL;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(swiglu_bf16_kernel, dim3(host_ceil_div(MI, kThreads), (unsigned)std::min<long>(rows, 65535)),
                     dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)gu, ldgu, (uint16_t*)act, rows, MI);
  return (int)hipGetLastError();
}

int qmoe_shared_gate(const void* sh, const void* gate, long ldg, void* out, long rows, int H, void* stream) {
  if (rows < 0 || H < 1 || ldg < 1) return QMOE_EINVAL;
  if (rows == 0) return 0;
  if (H % 8 == 0 && ((uintptr_t)sh & 15) == 0 && ((uintptr_t)out & 15) == 0) {
    hipLaunchKernelGGL(shared_gate_vec_kernel, dim3(host_ceil_div(H / 8, kThreads), (unsigned)std::min<long>(rows, 65535)),
                       dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)sh, (const uint16_t*)gate, ldg,
                       (uint16_t*)out, rows, H);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(shared_gate_kernel, dim3(host_ceil_div(H, kThreads), (unsigned)std::min<long>(rows, 65535)),
                     dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)sh, (const uint16_t*)gate, ldg,
                     (uint16_t*)out, rows, H);
  return (int)hipGetLastError();
}

}  // extern "C"
