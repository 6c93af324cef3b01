// Element-wise and byte-movement kernels around the expert GEMMs. Each keeps
// the reference's bf16 rounding points, so results are bit-exact with the CPU
// oracle for identical inputs.
#include "qmoe_common.h"
#include "qmoe.h"

#include <algorithm>

namespace {

// ow[kk, j*N/8 + c] = w4[ids[j], kk, c];  os[g, j*N + n] = S[ids[j], g, n]
// (kernels/expert_gather/gather.cpp:8-21). The source weight row (e, kk)
// starts at vector e * w_es + kk * w_rs: expert-major [E,K,N/8] has w_es =
// K * N/32, w_rs = N/32; K-major [K,E,N/8] has w_es = N/32, w_rs = E * N/32.
// Copies 16-byte vectors; an id outside [0, E) yields zero rows.
__global__ __launch_bounds__(256) void expert_gather_kernel(const uint4* __restrict__ w, const uint4* __restrict__ s,
                                                            const int64_t* __restrict__ ids, uint4* __restrict__ ow,
                                                            uint4* __restrict__ os, int K, int G, int N, int E,
                                                            int k, long w_es, long w_rs) {
  const int j = blockIdx.y;
  const int64_t e = ids[j];
  const bool ok = e >= 0 && e < E;
  const int wv = N / 32;  // 16-byte vectors per weight row (N/2 bytes)
  const int sv = N / 8;   // 16-byte vectors per scale row (2N bytes)
  const long wtot = (long)K * wv, stot = (long)G * sv;
  for (long q = (long)blockIdx.x * 256 + threadIdx.x; q < wtot + stot; q += (long)gridDim.x * 256) {
    if (q < wtot) {
      const long r = q / wv, c = q % wv;
      ow[(r * k + j) * wv + c] = ok ? w[e * w_es + r * w_rs + c] : make_uint4(0, 0, 0, 0);
    } else {
      const long q2 = q - wtot;
      const long r = q2 / sv, c = q2 % sv;
      os[(r * k + j) * sv + c] = ok ? s[((long)e * G + r) * sv + c] : make_uint4(0, 0, 0, 0);
    }
  }
}

// Weighted reduce, modes 1/2 (kernels/reduce/reduce.cpp:27-56): one thread
// per (token, column): acc = sum_g bf16(x[row] * w[t, g]) in order.
__global__ __launch_bounds__(256) void weighted_reduce_kernel(const uint16_t* __restrict__ x, const float* __restrict__ w,
                                                              const int64_t* __restrict__ inverse,
                                                              uint16_t* __restrict__ out, int B, int G, int W,
                                                              long row_stride, long nrows) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= W) return;
  for (long t = blockIdx.y; t < B; t += gridDim.y) {
    float acc = 0.f;
    for (int gi = 0; gi < G; ++gi) {
      const long row = inverse != nullptr ? inverse[t * G + gi] : t * G + gi;
      float v = 0.f;
      if (row >= 0 && row < nrows) v = bf16_to_f32(x[row * row_stride + col]);
      acc += round_bf16(v * w[t * G + gi]);
    }
    out[t * W + col] = (uint16_t)f32_to_bf16(acc);
  }
}

// The same sum on 8 columns per thread (16-byte loads) with every row of the
// token in flight together: rows of 8-aligned width and stride, G <= KMAX.
// Each column's terms are added in group order as above (the same bits).
// The products are read once: nontemporal loads.
template <int KMAX>
__global__ __launch_bounds__(1024) void weighted_reduce_vec_kernel(const uint16_t* __restrict__ x,
                                                                   const float* __restrict__ w,
                                                                   const int64_t* __restrict__ inverse,
                                                                   uint16_t* __restrict__ out, int B, int G, int W,
                                                                   long row_stride, long nrows) {
  const int c8 = blockIdx.x * blockDim.x + threadIdx.x;  // group of 8 columns
  if (8 * c8 >= W) return;
  for (long t = blockIdx.y; t < B; t += gridDim.y) {
    long rows[KMAX];
    float wt[KMAX];
#pragma unroll
    for (int gi = 0; gi < KMAX; ++gi) {
      rows[gi] = -1;
      wt[gi] = 0.f;
      if (gi < G) {
        rows[gi] = inverse != nullptr ? inverse[t * G + gi] : t * G + gi;
        wt[gi] = w[t * G + gi];
      }
    }
    uint4 v[KMAX];
#pragma unroll
    for (int gi = 0; gi < KMAX; ++gi)
      v[gi] = (gi < G && rows[gi] >= 0 && rows[gi] < nrows) ? load_nt16(x + rows[gi] * row_stride + 8 * c8)
                                                            : make_uint4(0u, 0u, 0u, 0u);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gi = 0; gi < KMAX; ++gi) {
      if (gi < G) {
        const uint32_t vv[4] = {v[gi].x, v[gi].y, v[gi].z, v[gi].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += round_bf16(bf16_to_f32(vv[q] & 0xffffu) * wt[gi]);
          acc[2 * q + 1] += round_bf16(bf16_to_f32(vv[q] >> 16) * wt[gi]);
        }
      }
    }
    uint32_t r[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = f32_to_bf16(acc[q]);
    *reinterpret_cast<uint4*>(out + t * W + 8 * c8) =
        make_uint4(r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16), r[6] | (r[7] << 16));
  }
}

// Decode epilogue over the Cartesian down output (kernels/moe_epilogue/epilogue.cpp:17-39):
// r = bf16(sum_j bf16(y[j, j*H + n] * w_j)); out = bf16(r + bf16(sh * bf16(sigmoid(gate)))).
__global__ __launch_bounds__(256) void moe_epilogue_kernel(const uint16_t* __restrict__ cart,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ shared,
                                                           const uint16_t* __restrict__ gate,
                                                           uint16_t* __restrict__ out, int k, int H) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= H) return;
  float acc = 0.f;
  for (int j = 0; j < k; ++j)
    acc += round_bf16(bf16_to_f32(cart[(long)j * k * H + (long)j * H + n]) * bf16_to_f32(w[j]));
  float r = round_bf16(acc);
  if (shared != nullptr) {
    const float sg = round_bf16(1.0f / (1.0f + expf(-bf16_to_f32(gate[0]))));
    r = round_bf16(r + round_bf16(bf16_to_f32(shared[n]) * sg));
  }
  out[n] = (uint16_t)f32_to_bf16(r);
}

// Shared-expert merge (kernels/post_ops/post_ops.cpp:72-94):
// out = bf16(e + bf16(s * bf16(sigmoid(g_t)))), one gate value per row.
__global__ __launch_bounds__(256) void moe_merge_kernel(const uint16_t* __restrict__ e, const uint16_t* __restrict__ s,
                                                        const uint16_t* __restrict__ gate, uint16_t* __restrict__ out,
                                                        int B, int W) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= W) return;
  for (long t = blockIdx.y; t < B; t += gridDim.y) {
    const float sg = round_bf16(1.0f / (1.0f + expf(-bf16_to_f32(gate[t]))));
    const long o = t * W + n;
    out[o] = (uint16_t)f32_to_bf16(bf16_to_f32(e[o]) + round_bf16(bf16_to_f32(s[o]) * sg));
  }
}

// act = bf16(silu(fp32 g) * fp32 u); g = first MI columns, u = last MI
// (npu_swiglu on fp32 input then .to(bf16), fnx/engine.py:1827,1866).
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ act,
                                                     long rows, int MI) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= MI) return;
  for (long r = blockIdx.y; r < rows; r += gridDim.y) {
    const float gv = bf16_to_f32(gu[r * 2 * MI + i]);
    const float uv = bf16_to_f32(gu[r * 2 * MI + MI + i]);
    act[r * MI + i] = (uint16_t)f32_to_bf16(silu_f32(gv) * uv);
  }
}

// The same merge and SwiGLU on 8 elements per thread (16-byte accesses) for
// 8-aligned widths and 16-byte aligned tensors; the same arithmetic per
// element (the same bits).
__global__ __launch_bounds__(256) void moe_merge_vec_kernel(const uint16_t* __restrict__ e, const uint16_t* __restrict__ s,
                                                            const uint16_t* __restrict__ gate,
                                                            uint16_t* __restrict__ out, int B, int W) {
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  if (8 * c8 >= W) return;
  for (long t = blockIdx.y; t < B; t += gridDim.y) {
    const float sg = round_bf16(1.0f / (1.0f + expf(-bf16_to_f32(gate[t]))));
    const long o = t * W + 8 * c8;
    const uint4 ev = *reinterpret_cast<const uint4*>(e + o), sv = *reinterpret_cast<const uint4*>(s + o);
    const uint32_t ew[4] = {ev.x, ev.y, ev.z, ev.w}, sw[4] = {sv.x, sv.y, sv.z, sv.w};
    uint32_t r[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = f32_to_bf16(bf16_to_f32(ew[q] & 0xffffu) + round_bf16(bf16_to_f32(sw[q] & 0xffffu) * sg));
      const uint32_t hi = f32_to_bf16(bf16_to_f32(ew[q] >> 16) + round_bf16(bf16_to_f32(sw[q] >> 16) * sg));
      r[q] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(out + o) = make_uint4(r[0], r[1], r[2], r[3]);
  }
}

__global__ __launch_bounds__(256) void swiglu_vec_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ act,
                                                         long rows, int MI) {
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  if (8 * c8 >= MI) return;
  for (long r = blockIdx.y; r < rows; r += gridDim.y) {
    const uint4 gv = *reinterpret_cast<const uint4*>(gu + r * 2 * MI + 8 * c8);
    const uint4 uv = *reinterpret_cast<const uint4*>(gu + r * 2 * MI + MI + 8 * c8);
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = f32_to_bf16(silu_f32(bf16_to_f32(gw[q] & 0xffffu)) * bf16_to_f32(uw[q] & 0xffffu));
      const uint32_t hi = f32_to_bf16(silu_f32(bf16_to_f32(gw[q] >> 16)) * bf16_to_f32(uw[q] >> 16));
      o[q] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(act + r * MI + 8 * c8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

bool aligned16_ptr(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

static int gather_launch(const void* w4, const void* scales, const void* ids, void* ow, void* os, int K, int G,
                         int N, int E, int k, bool expert_major, void* stream) {
  if (K < 1 || G < 1 || N < 32 || (N % 32) || E < 1 || k < 1 || k > 65535) return QMOE_EINVAL;
  const long wv = N / 32;
  const long tot = (long)K * wv + (long)G * (N / 8);
  const int bx = (int)std::min<long>((tot + 255) / 256, 1024);
  const long w_es = expert_major ? (long)K * wv : wv, w_rs = expert_major ? wv : (long)E * wv;
  hipLaunchKernelGGL(expert_gather_kernel, dim3(bx, k), dim3(256), 0, (hipStream_t)stream, (const uint4*)w4,
                     (const uint4*)scales, (const int64_t*)ids, (uint4*)ow, (uint4*)os, K, G, N, E, k, w_es, w_rs);
  return (int)hipGetLastError();
}

int qmoe_expert_gather(const void* w4, const void* scales, const void* ids, void* ow, void* os, int K, int G,
                       int N, int E, int k, void* stream) {
  return gather_launch(w4, scales, ids, ow, os, K, G, N, E, k, true, stream);
}

int qmoe_expert_gather_kmajor(const void* w4, const void* scales, const void* ids, void* ow, void* os, int K, int G,
                              int N, int E, int k, void* stream) {
  return gather_launch(w4, scales, ids, ow, os, K, G, N, E, k, false, stream);
}

int qmoe_weighted_reduce(const void* x, const void* w_f32, const void* inverse, void* out, int B, int G, int W,
                         long row_stride, long nrows, void* stream) {
  if (B < 1 || G < 1 || W < 1 || row_stride < W || nrows < 1) return QMOE_EINVAL;
  if (G <= QMOE_KMAX && (W % 8) == 0 && (row_stride % 8) == 0 && ((uintptr_t)x & 15) == 0 &&
      ((uintptr_t)out & 15) == 0) {
    // one row of W/8 threads per token (up to 1024), every product row in flight
    const int threads = std::min(1024, host_ceil_div(W / 8, 64) * 64);
    hipLaunchKernelGGL(weighted_reduce_vec_kernel<QMOE_KMAX>, dim3(host_ceil_div(W / 8, threads), std::min(B, 65535)),
                       dim3(threads), 0, (hipStream_t)stream, (const uint16_t*)x, (const float*)w_f32,
                       (const int64_t*)inverse, (uint16_t*)out, B, G, W, row_stride, nrows);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(weighted_reduce_kernel, dim3(host_ceil_div(W, 256), std::min(B, 65535)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const float*)w_f32, (const int64_t*)inverse, (uint16_t*)out, B, G, W,
                     row_stride, nrows);
  return (int)hipGetLastError();
}

int qmoe_moe_epilogue(const void* cart, const void* w, const void* shared, const void* gate, void* out, int k,
                      int H, void* stream) {
  if (k < 1 || H < 1 || (shared == nullptr) != (gate == nullptr)) return QMOE_EINVAL;
  hipLaunchKernelGGL(moe_epilogue_kernel, dim3(host_ceil_div(H, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)cart, (const uint16_t*)w, (const uint16_t*)shared, (const uint16_t*)gate,
                     (uint16_t*)out, k, H);
  return (int)hipGetLastError();
}

int qmoe_moe_merge(const void* e, const void* s, const void* gate, void* out, int B, int W, void* stream) {
  if (B < 1 || W < 1) return QMOE_EINVAL;
  if ((W % 8) == 0 && aligned16_ptr(e) && aligned16_ptr(s) && aligned16_ptr(out)) {
    hipLaunchKernelGGL(moe_merge_vec_kernel, dim3(host_ceil_div(W / 8, 256), std::min(B, 65535)), dim3(256), 0,
                       (hipStream_t)stream, (const uint16_t*)e, (const uint16_t*)s, (const uint16_t*)gate,
                       (uint16_t*)out, B, W);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(moe_merge_kernel, dim3(host_ceil_div(W, 256), std::min(B, 65535)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)e, (const uint16_t*)s, (const uint16_t*)gate, (uint16_t*)out, B, W);
  return (int)hipGetLastError();
}

int qmoe_swiglu(const void* gu, void* act, int rows, int MI, void* stream) {
  if (rows < 0 || MI < 1) return QMOE_EINVAL;
  if (rows == 0) return 0;
  if ((MI % 8) == 0 && aligned16_ptr(gu) && aligned16_ptr(act)) {
    hipLaunchKernelGGL(swiglu_vec_kernel, dim3(host_ceil_div(MI / 8, 256), std::min(rows, 65535)), dim3(256), 0,
                       (hipStream_t)stream, (const uint16_t*)gu, (uint16_t*)act, (long)rows, MI);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(swiglu_kernel, dim3(host_ceil_div(MI, 256), std::min(rows, 65535)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)gu, (uint16_t*)act, (long)rows, MI);
  return (int)hipGetLastError();
}

}  // extern "C"
