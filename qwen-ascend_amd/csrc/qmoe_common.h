// Shared device helpers for the qmoe HIP kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QMOE_DEV __device__ __forceinline__
#define QMOE_HOST_DEV __host__ __device__ __forceinline__

// Return codes of every extern "C" entry point.
enum {
  QMOE_OK = 0,
  QMOE_EINVAL = -1,      // shape / size / alignment rejected before launch
  QMOE_EWORKSPACE = -2,  // caller-provided workspace too small
  QMOE_ESCRATCH = -3,    // shape needs more than a fixed no-allocation scratch holds
};

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));

// 16-byte load of data read once (weights of a streaming pass): marked
// nontemporal, so its lines do not displace the reused data in the caches.
QMOE_DEV uint4 load_nt16(const void* p) {
  const u32x4_v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------- bf16 <-> f32

QMOE_DEV float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Round-to-nearest-even to bf16, NaN kept quiet with its payload top bits.
// Bit-identical to the oracle's f32_to_bf16_bits.
QMOE_DEV uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  // a select, not a branch: both forms are a few operations
  return ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : rne;
}

QMOE_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// silu(g) = g * sigmoid(g) in fp32, from y = e^-|g| in (0, 1]: sigmoid =
// 1/(1+y) for g >= 0 and y/(1+y) below, so nothing overflows. Hardware exp2
// and reciprocal: a few fp32 ulps, far inside the bf16 rounding that follows.
// Every kernel (decode, prefill epilogue, the standalone SwiGLU) uses this
// one form, so the fused and the unfused paths round identically.
QMOE_DEV float silu_f32(float g) {
  const float y = __builtin_amdgcn_exp2f(-fabsf(g) * 1.44269504088896341f);
  const float r = __builtin_amdgcn_rcpf(1.0f + y);
  return g * (g >= 0.0f ? r : y * r);
}

// bf16(bf16(silu(g)) * u) for bf16 bit patterns g, u: the two roundings of
// F.silu(g) * u on bf16 tensors.
QMOE_DEV uint32_t swiglu_bf16_bits(uint32_t g, uint32_t u) {
  const float s = bf16_to_f32(f32_to_bf16(silu_f32(bf16_to_f32(g))));
  return f32_to_bf16(s * bf16_to_f32(u));
}

// Monotone 16-bit key of a bf16 pattern (larger value -> larger key).
QMOE_DEV uint32_t bf16_order_key(uint32_t b) {
  return (b & 0x8000u) ? ((~b) & 0xffffu) : (b | 0x8000u);
}
QMOE_DEV uint32_t bf16_from_order_key(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7fffu) : ((~k) & 0xffffu);
}

// ---------------------------------------------------------------- wave64 reductions (DPP)

// DPP row operations below use bound_ctrl with full row and bank masks:
// every lane is written and the source lane always exists (quad
// permutations and row mirrors), so the compiler folds each move into the
// max or add that consumes it.
#define QMOE_DPP(v, ctrl) ((uint32_t)__builtin_amdgcn_mov_dpp((int)(v), (ctrl), 0xf, 0xf, true))
#define QMOE_DPPF(v, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), (ctrl), 0xf, 0xf, true))

// Max over the 64 lanes of a wave, result uniform in every lane.
QMOE_DEV uint32_t wave_max_u32(uint32_t v) {
  // quad butterflies (xor 1, xor 2), then half-row and row mirrors: every lane
  // of a 16-lane row holds the row max.
  v = max(v, QMOE_DPP(v, 0xB1));
  v = max(v, QMOE_DPP(v, 0x4E));
  v = max(v, QMOE_DPP(v, 0x141));
  v = max(v, QMOE_DPP(v, 0x140));
  uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// Sum over the 64 lanes of a wave in a fixed tree order, result uniform.
QMOE_DEV float wave_sum_f32(float v) {
  v += QMOE_DPPF(v, 0xB1);
  v += QMOE_DPPF(v, 0x4E);
  v += QMOE_DPPF(v, 0x141);
  v += QMOE_DPPF(v, 0x140);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

// ---------------------------------------------------------------- routing (top-k)

// Largest supported top-k.
#define QMOE_KMAX 16

// Full-wave maximum left in every lane, with no scalar round trip: row
// maxima by DPP, then the row pairs (1<->0, 3<->2) and halves swapped by
// v_permlane16_swap / v_permlane32_swap.
QMOE_DEV uint32_t wave_max_u32_vec(uint32_t v) {
  v = max(v, QMOE_DPP(v, 0xB1));
  v = max(v, QMOE_DPP(v, 0x4E));
  v = max(v, QMOE_DPP(v, 0x141));
  v = max(v, QMOE_DPP(v, 0x140));
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)a[0], (uint32_t)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)b[0], (uint32_t)b[1]);
}

// Top-k over one token's logits by one full wave, in three steps.
// Selection key: larger logit, then lower expert id (the key packs the bf16
// order key above the inverted id, so all keys are distinct and nonzero).
//
// wave_route_keys: lane l holds logits l*KPL .. l*KPL+KPL-1 (keys, and the
// logits as fp32; -inf / key 0 past E). E <= 64 * KPL.
//
// route_load_vec / route_keys_vec are its two halves for whole 16-byte
// groups (KPL % 8 == 0, E % 8 == 0, logits 16-byte aligned): one vector load
// per 8 logits, issued by every lane (lanes past E re-read the last group),
// so a kernel can put the load out early and form the keys later.
template <int KPL>
QMOE_DEV void route_load_vec(const uint16_t* __restrict__ logits, int E, uint4* raw) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < KPL; i += 8) raw[i / 8] = *reinterpret_cast<const uint4*>(logits + min(lane * KPL + i, E - 8));
}
template <int KPL>
QMOE_DEV void route_keys_of(const uint32_t* raw, int E, uint32_t* key, float* lg) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = lane * KPL + i;
    if (e < E) {
      key[i] = (bf16_order_key(raw[i]) << 16) | (0xffffu - (uint32_t)e);
      lg[i] = bf16_to_f32(raw[i]);
    } else {
      key[i] = 0u;
      lg[i] = -INFINITY;
    }
  }
}
template <int KPL>
QMOE_DEV void route_keys_vec(const uint4* rv, int E, uint32_t* key, float* lg) {
  uint32_t raw[KPL];
#pragma unroll
  for (int i = 0; i < KPL / 8; ++i) {
    const uint32_t vv[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      raw[8 * i + 2 * q] = vv[q] & 0xffffu;
      raw[8 * i + 2 * q + 1] = vv[q] >> 16;
    }
  }
  route_keys_of<KPL>(raw, E, key, lg);
}
template <int KPL>
QMOE_DEV void wave_route_keys(const uint16_t* __restrict__ logits, int E, uint32_t* key, float* lg) {
  if (KPL % 8 == 0 && (E % 8) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15u) == 0) {
    uint4 rv[KPL / 8 > 0 ? KPL / 8 : 1];
    route_load_vec<KPL>(logits, E, rv);
    route_keys_vec<KPL>(rv, E, key, lg);
  } else {
    const int lane = threadIdx.x & 63;
    uint32_t raw[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) raw[i] = (lane * KPL + i < E) ? (uint32_t)logits[lane * KPL + i] : 0u;
    route_keys_of<KPL>(raw, E, key, lg);
  }
}

#define QMOE_CE(a, b)                               \
  {                                                 \
    const uint32_t hi_ = max(a, b), lo_ = min(a, b); \
    a = hi_;                                        \
    b = lo_;                                        \
  }

// wave_route_select: returns, in lane r < k, the key of rank r (0 in the
// other lanes). KPL == 8: each lane sorts its keys (Batcher's 19-comparator
// network) and every round takes the wave maximum of the list heads; the
// lane that held it pops its head. Otherwise every round takes the wave
// maximum over all keys and clears it. Both give the same keys (they are
// distinct). The rounds are a rolled loop: a wave runs this code once per
// launch, so its length, not its trip count, sets the cost of fetching it.
//
// RouteSelect holds the state between rounds, so a wave can take the first
// ranks, hand them on, and take the rest later (rank r is fixed after round
// r, whatever follows).
template <int KPL>
struct RouteSelect {
  uint32_t a[KPL];
  uint32_t mine;
  QMOE_DEV void init(const uint32_t* key) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) a[i] = key[i];
    if constexpr (KPL == 8) {
      QMOE_CE(a[0], a[1]); QMOE_CE(a[2], a[3]); QMOE_CE(a[4], a[5]); QMOE_CE(a[6], a[7]);
      QMOE_CE(a[0], a[2]); QMOE_CE(a[1], a[3]); QMOE_CE(a[4], a[6]); QMOE_CE(a[5], a[7]);
      QMOE_CE(a[1], a[2]); QMOE_CE(a[5], a[6]);
      QMOE_CE(a[0], a[4]); QMOE_CE(a[1], a[5]); QMOE_CE(a[2], a[6]); QMOE_CE(a[3], a[7]);
      QMOE_CE(a[2], a[4]); QMOE_CE(a[3], a[5]);
      QMOE_CE(a[1], a[2]); QMOE_CE(a[3], a[4]); QMOE_CE(a[5], a[6]);
    }
    mine = 0u;
  }
  // ranks r0 .. r1 - 1
  QMOE_DEV void rounds(int r0, int r1) {
    const int lane = threadIdx.x & 63;
#pragma unroll 1
    for (int r = r0; r < r1; ++r) {
      uint32_t best;
      if constexpr (KPL == 8) {
        best = wave_max_u32_vec(a[0]);
        const bool w = a[0] == best;
#pragma unroll
        for (int i = 0; i < 7; ++i) a[i] = w ? a[i + 1] : a[i];
        a[7] = w ? 0u : a[7];
      } else {
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < KPL; ++i) m = max(m, a[i]);
        best = wave_max_u32(m);
#pragma unroll
        for (int i = 0; i < KPL; ++i) a[i] = (a[i] == best) ? 0u : a[i];
      }
      mine = (lane == r) ? best : mine;
    }
  }
};

template <int KPL>
QMOE_DEV uint32_t wave_route_select(uint32_t* key, int k) {
  RouteSelect<KPL> rs;
  rs.init(key);
  rs.rounds(0, k);
  return rs.mine;
}

// Key of rank r (r wave-uniform) of a selection held one rank per lane.
QMOE_DEV uint32_t route_sel_rank(uint32_t sel_lane, int r) {
  return (uint32_t)__builtin_amdgcn_readlane((int)sel_lane, r);
}

// Expert id of a selection key.
QMOE_DEV int route_key_expert(uint32_t key) { return (int)(0xffffu - (key & 0xffffu)); }

// wave_route_softmax: lane r < k writes idx_out[r] and the renormalised
// softmax probability w_out[r] (fp32, before the final bf16 rounding): p_r =
// exp(l_r - max) / Z with Z summed over all E in a fixed tree order, w_r =
// p_r / (p_0 + ... + p_{k-1}) summed in rank order. sel_lane is the
// selection of wave_route_select (lane r holds the key of rank r).
template <int KPL>
QMOE_DEV void wave_route_softmax(const float* lg, int E, int k, uint32_t sel_lane, int* idx_out, float* w_out) {
  const int lane = threadIdx.x & 63;
  const float mx = bf16_to_f32(bf16_from_order_key(route_sel_rank(sel_lane, 0) >> 16));
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < KPL; ++i) z += (lane * KPL + i < E) ? __expf(lg[i] - mx) : 0.f;
  z = wave_sum_f32(z);
  const float p = (lane < k) ? __expf(bf16_to_f32(bf16_from_order_key(sel_lane >> 16)) - mx) / z : 0.f;
  float s = 0.f;
#pragma unroll 1
  for (int r = 0; r < k; ++r) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), r));
  if (lane < k) {
    idx_out[lane] = route_key_expert(sel_lane);
    w_out[lane] = p / s;
  }
}

// All three: top-k of one token's logits by one wave. k <= QMOE_KMAX.
template <int KPL>
QMOE_DEV void wave_topk_softmax(const uint16_t* __restrict__ logits, int E, int k,
                                int* idx_out, float* w_out) {
  uint32_t key[KPL];
  float lg[KPL];
  wave_route_keys<KPL>(logits, E, key, lg);
  const uint32_t sel = wave_route_select<KPL>(key, k);
  wave_route_softmax<KPL>(lg, E, k, sel, idx_out, w_out);
}

// ---------------------------------------------------------------- cross-workgroup hand-off
//
// Partial results that another workgroup of the same launch reduces are
// written and read with agent-scope (sc1) accesses, which go through to the
// device-coherent level instead of the per-XCD L2. An arriving workgroup
// waits for its own stores to complete, then bumps an arrival counter; the
// last arriver reads everyone's partials. No L2 write-back/invalidate
// (__threadfence) is needed.

QMOE_DEV void store_agent(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// 64-bit device-coherent accesses (single-copy atomic when 8-byte aligned):
// a value travels with its tag in one word.
QMOE_DEV void store_agent64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
QMOE_DEV uint64_t load_agent64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
QMOE_DEV float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// sum_{i < n} p[i * stride] in index order. The device-coherent loads are
// issued BATCH at a time before any is used (indexes past n re-read the last
// element and are not added), so a reduction costs about n / BATCH memory
// round trips instead of n.
template <int BATCH = 8>
QMOE_DEV float sum_agent_ordered(const float* p, size_t stride, int n) {
  float s = 0.f;
  for (int b = 0; b < n; b += BATCH) {
    float v[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) v[i] = load_agent(p + (size_t)min(b + i, n - 1) * stride);
#pragma unroll
    for (int i = 0; i < BATCH; ++i)
      if (b + i < n) s += v[i];
  }
  return s;
}

// Returns true (uniformly) in the workgroup that arrives last at `counter`
// out of `total`; that workgroup resets the counter to zero for the next
// launch. Every thread's agent-scope stores complete before the arrival.
// v, made to depend on t through an empty asm: an operation that uses the
// result waits until t is available (a counter bump that must follow the
// load of t, whatever the memory system does with two addresses).
QMOE_DEV int after(uint32_t t, int v) {
  asm volatile("" : "+v"(v) : "v"(t));
  return v;
}

// Two-level arrival count, thread 0 of a workgroup: the workgroup counts
// itself on its group's counter; the last of a group counts the group on the
// top counter (a workgroup with no group counter counts there directly); the
// last count on the top counter stores `tag` to the epoch. Every counter is
// left at zero. Atomics on one address are served one after another, so
// spreading a launch's counts over several counters (128 bytes apart) keeps
// the wait for each count short. The first count waits for `tag`, so it
// follows the load of the epoch.
QMOE_DEV void arrive2(int* group_ctr, int group_total, int* top_ctr, int top_total, uint32_t* epoch, uint32_t tag) {
  const int one = after(tag, 1);
  if (group_ctr != nullptr) {
    if (__hip_atomic_fetch_add(group_ctr, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != group_total - 1) return;
    __hip_atomic_store(group_ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (__hip_atomic_fetch_add(top_ctr, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != top_total - 1) return;
  __hip_atomic_store(epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(top_ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

QMOE_DEV bool arrive_last(int* counter, int total) {
  __shared__ int s_prev;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) s_prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const bool last = (s_prev == total - 1);
  if (last && threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// ---------------------------------------------------------------- misc

QMOE_DEV int ceil_div(int a, int b) { return (a + b - 1) / b; }
static inline int host_ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// Map a launch-order block id to a logical tile id so that consecutive
// logical tiles run on the same XCD (blocks are dealt round-robin over the
// 8 XCDs of an MI355X). Keeps tiles that share operands in one L2.
QMOE_DEV int xcd_remap(int bid, int nblocks) {
  const int nx = 8;
  const int per = nblocks / nx;          // full rounds
  const int rem = nblocks - per * nx;    // leftover blocks in the last round
  const int x = bid % nx, i = bid / nx;
  if (i >= per) return bid;              // last partial round: identity
  // XCD x owns logical ids [x*per, (x+1)*per) among the first per*nx
  (void)rem;
  return x * per + i;
}
