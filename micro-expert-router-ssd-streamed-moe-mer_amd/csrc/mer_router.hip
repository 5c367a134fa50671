// mer_router.hip -- LinearGate routing on the GPU for gfx950.
//
// Two launches restate LinearGate::route_with_scratch
// (gating.rs:395-476) with its full routing surface (with_routing,
// gating.rs:207-268):
//   logits    = W x                               (W: [n_experts][d_model] f32)
//               router_logits_kernel: one wave per (expert, group of 4
//               tokens), so the gate matrix streams through every CU
//               with many loads in flight (one token reads all of W);
//   the rest, one 256-thread workgroup per token (router_kernel):
//   scores    = softmax(logits) (transformer.rs:2807, non-finite rows fall
//               back to uniform) or sigmoid (gating.rs:271-279)
//   selection = scores + correction_bias          (bias optional)
//   optional group filter (gating.rs:321-370): groups scored by the sum of
//               their two best selection scores, the best topk_group survive
//   top-k over surviving experts with finite selection (higher first, lower
//               id on ties; insert_top_expert, gating.rs:296-320)
//   weights   = unbiased scores at the chosen experts, renormalised when
//               their sum is finite and > 0, then scaled.
// The dot products are f32 with a different summation order from the
// reference's matvec, so logits agree to f32 rounding, not bit for bit.
#include "mer_internal.hpp"

namespace mer {

namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / 64;
constexpr uint32_t kRouterTokGroup = 4;  // tokens per logits wave
// The per-token selection runs as one wave: its reductions are shuffles and
// its barriers cost no waiting on other waves.
constexpr int kSelThreads = 64;
constexpr int kSelWaves = 1;

// Total order of f32 (f32::total_cmp) as a signed integer key.
__device__ __forceinline__ int32_t total_key(float v) {
  const int32_t b = __float_as_int(v);
  return b ^ ((b >> 31) & 0x7fffffff);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Candidate (key, id) comparison: better = larger key, then smaller id.
__device__ __forceinline__ bool better(int32_t ka, int32_t ia, int32_t kb, int32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// (key, id) as one unsigned 64-bit value ordered like `better`: the key with
// its sign bit flipped above the complemented id.  0 is below every
// candidate (a real one has a complemented id >= 2^32 - 1024).
__device__ __forceinline__ uint64_t pack_candidate(int32_t key, uint32_t id) {
  return ((uint64_t)((uint32_t)key ^ 0x80000000u) << 32) | (uint64_t)(0xffffffffu - id);
}

// Largest packed candidate of the wave, in every lane: DPP row rotations
// (8, 4, 2, 1) give each lane its row's maximum, then the four row maxima
// are read out.  No LDS-routed permutes on the path.
__device__ __forceinline__ uint64_t wave_max_candidate(uint64_t v) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
#define MER_ROW_ROR_MAX(CTRL)                                                                     \
  {                                                                                               \
    const uint32_t l2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, 0xf, 0xf, false); \
    const uint32_t h2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, 0xf, 0xf, false); \
    if (h2 > hi || (h2 == hi && l2 > lo)) {                                                       \
      hi = h2;                                                                                    \
      lo = l2;                                                                                    \
    }                                                                                             \
  }
  MER_ROW_ROR_MAX(0x128)
  MER_ROW_ROR_MAX(0x124)
  MER_ROW_ROR_MAX(0x122)
  MER_ROW_ROR_MAX(0x121)
#undef MER_ROW_ROR_MAX
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t c = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)hi, 16 * r) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)lo, 16 * r);
    best = c > best ? c : best;
  }
  return best;
}

}  // namespace

// logit_buf[t][e] = W[e] . x[t] for a group of up to 4 tokens per wave.
// VEC: 16-byte loads (d_model % 4 == 0 and 16-byte aligned gate and x).
template <bool VEC>
__global__ __launch_bounds__(kRouterThreads) void router_logits_kernel(RouterParams p) {
  const uint32_t n_eg = (p.n_experts + kRouterWaves - 1) / kRouterWaves;
  const uint32_t eg = blockIdx.x % n_eg, tg = blockIdx.x / n_eg;
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t e = eg * kRouterWaves + wave;
  if (e >= p.n_experts) return;  // the whole wave; nothing below synchronises the workgroup
  const uint32_t t0 = tg * kRouterTokGroup;
  const uint32_t nt = min(kRouterTokGroup, p.n_tokens - t0);
  const float *w = p.gate + (size_t)e * p.d_model;
  const float *x = p.x + (size_t)t0 * p.d_model;
  float acc[kRouterTokGroup] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (VEC) {
#pragma unroll 8
    for (uint32_t d = 4 * lane; d < p.d_model; d += 256) {
      const float4 wv = *reinterpret_cast<const float4 *>(w + d);
#pragma unroll
      for (uint32_t j = 0; j < kRouterTokGroup; ++j)
        if (j < nt) {
          const float4 xv = *reinterpret_cast<const float4 *>(x + (size_t)j * p.d_model + d);
          acc[j] = __builtin_fmaf(wv.x, xv.x, acc[j]);
          acc[j] = __builtin_fmaf(wv.y, xv.y, acc[j]);
          acc[j] = __builtin_fmaf(wv.z, xv.z, acc[j]);
          acc[j] = __builtin_fmaf(wv.w, xv.w, acc[j]);
        }
    }
  } else {
#pragma unroll 8
    for (uint32_t d = lane; d < p.d_model; d += 64) {
      const float wv = w[d];
#pragma unroll
      for (uint32_t j = 0; j < kRouterTokGroup; ++j)
        if (j < nt) acc[j] = __builtin_fmaf(wv, x[(size_t)j * p.d_model + d], acc[j]);
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < kRouterTokGroup; ++j) {
    const float v = wave_sum(acc[j]);
    if (lane == 0 && j < nt) p.logit_buf[(size_t)(t0 + j) * p.n_experts + e] = v;
  }
}

__global__ __launch_bounds__(kSelThreads) void router_kernel(RouterParams p) {
  extern __shared__ float smem[];
  float *scores = smem;                               // [n_experts]
  float *selection = scores + p.n_experts;            // [n_experts]
  __shared__ float red_f[kSelWaves];
  __shared__ uint32_t group_ok[kMaxRouterExperts / 32];
  __shared__ int32_t chosen[kMaxRouterTopK];
  // thread 0's working arrays, in LDS (as private arrays they would live in
  // scratch memory, whose set-up dominates a launch this small)
  __shared__ int32_t sel_g[kMaxRouterGroups];  // surviving groups, best first
  __shared__ float sel_s[kMaxRouterGroups];
  __shared__ float w[kMaxRouterTopK];
  __shared__ int32_t flag_bad;

  const uint32_t t = blockIdx.x;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  if (tid == 0) flag_bad = 0;
  // the token's logits, from router_logits_kernel
  for (uint32_t e = tid; e < p.n_experts; e += kSelThreads) scores[e] = p.logit_buf[(size_t)t * p.n_experts + e];
  __syncthreads();

  // ---- scores -------------------------------------------------------------
  if (p.scoring == 0) {
    // softmax: max over non-NaN values; a NaN or a non-finite max makes the
    // row uniform (softmax_inplace's fallback)
    float m = -INFINITY;
    for (uint32_t e = tid; e < p.n_experts; e += kSelThreads) {
      const float v = scores[e];
      if (v != v) flag_bad = 1;  // benign race: every writer stores 1
      else m = __builtin_fmaxf(m, v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = red_f[0];
    for (int i = 1; i < kSelWaves; ++i) m = __builtin_fmaxf(m, red_f[i]);
    const bool uniform = flag_bad || !__builtin_isfinite(m);
    __syncthreads();
    float s = 0.f;
    for (uint32_t e = tid; e < p.n_experts; e += kSelThreads) {
      const float v = uniform ? 1.f : expf(scores[e] - m);
      scores[e] = v;
      s += v;
    }
    s = wave_sum(s);
    if (lane == 0) red_f[wave] = s;
    __syncthreads();
    float sum = 0.f;
    for (int i = 0; i < kSelWaves; ++i) sum += red_f[i];
    for (uint32_t e = tid; e < p.n_experts; e += kSelThreads)
      scores[e] = uniform ? 1.0f / (float)p.n_experts : (sum > 0.f ? scores[e] / sum : scores[e]);
  } else {
    for (uint32_t e = tid; e < p.n_experts; e += kSelThreads) scores[e] = 1.0f / (1.0f + expf(-scores[e]));
  }
  __syncthreads();
  for (uint32_t e = tid; e < p.n_experts; e += kSelThreads)
    selection[e] = p.bias ? scores[e] + p.bias[e] : scores[e];
  for (uint32_t i = tid; i < kMaxRouterExperts / 32; i += kSelThreads) group_ok[i] = 0xffffffffu;
  __syncthreads();

  // ---- optional group filter ----------------------------------------------
  const bool grouped = p.n_group > 1 && p.topk_group > 0 && p.topk_group < p.n_group && p.n_experts % p.n_group == 0;
  if (grouped && tid == 0) {
    const uint32_t gs = p.n_experts / p.n_group;
    uint32_t c = 0;
    for (uint32_t g = 0; g < p.n_group; ++g) {
      float top1 = -INFINITY, top2 = -INFINITY;
      for (uint32_t i = 0; i < gs; ++i) {
        const float v = selection[g * gs + i];
        if (v > top1) {
          top2 = top1;
          top1 = v;
        } else if (v > top2) {
          top2 = v;
        }
      }
      const float sum = top1 + (__builtin_isfinite(top2) ? top2 : 0.0f);
      // insert_top_group: total order, lower id on ties, keep topk_group
      uint32_t pos = c;
      for (uint32_t i = 0; i < c; ++i)
        if (better(total_key(sum), (int32_t)g, total_key(sel_s[i]), sel_g[i])) {
          pos = i;
          break;
        }
      if (pos == c && c >= p.topk_group) continue;
      const uint32_t last = c < p.topk_group ? c : p.topk_group - 1;
      for (uint32_t i = last; i > pos; --i) {
        sel_g[i] = sel_g[i - 1];
        sel_s[i] = sel_s[i - 1];
      }
      sel_g[pos] = (int32_t)g;
      sel_s[pos] = sum;
      if (c < p.topk_group) ++c;
    }
    for (uint32_t i = 0; i < kMaxRouterExperts / 32; ++i) group_ok[i] = 0u;
    for (uint32_t i = 0; i < c; ++i)
      for (uint32_t e = (uint32_t)sel_g[i] * gs; e < ((uint32_t)sel_g[i] + 1) * gs; ++e) group_ok[e >> 5] |= 1u << (e & 31u);
  }
  __syncthreads();

  // ---- top-k: k rounds of a wave arg-max -------------------------------
  // Each round's winner (the largest packed candidate) is known to every
  // lane; each lane remembers which of its own experts (lane, lane + 64, ...)
  // are taken.
  static_assert(kSelThreads == 64 && kMaxRouterExperts <= 64 * 64, "one wave, a 64-bit taken mask per lane");
  uint64_t taken = 0;  // bit i: expert lane + 64 i is chosen
  uint32_t count = 0;
  for (uint32_t r = 0; r < p.top_k; ++r) {
    uint64_t mine = 0;
    uint32_t i = 0;
    for (uint32_t e = lane; e < p.n_experts; e += 64, ++i) {
      const float v = selection[e];
      if (!__builtin_isfinite(v) || !((group_ok[e >> 5] >> (e & 31u)) & 1u) || ((taken >> i) & 1u)) continue;
      const uint64_t c = pack_candidate(total_key(v), e);
      mine = c > mine ? c : mine;
    }
    const uint64_t best = wave_max_candidate(mine);
    if (best == 0) break;  // the same in every lane: no eligible expert left
    const uint32_t bi = 0xffffffffu - (uint32_t)best;
    if (lane == (bi & 63u)) taken |= 1ull << (bi >> 6);
    if (lane == 0) chosen[r] = (int32_t)bi;
    count = r + 1;
  }
  __syncthreads();

  // ---- weights ------------------------------------------------------------
  if (tid == 0) {
    float sum = 0.f;
    for (uint32_t i = 0; i < count; ++i) {
      w[i] = scores[chosen[i]];
      sum = sum + w[i];
    }
    if (p.normalise && __builtin_isfinite(sum) && sum > 0.f)
      for (uint32_t i = 0; i < count; ++i) w[i] = w[i] / sum;
    if (p.scaling != 1.0f && __builtin_isfinite(p.scaling))
      for (uint32_t i = 0; i < count; ++i) w[i] = w[i] * p.scaling;
    for (uint32_t i = 0; i < p.top_k; ++i) {
      p.ids[(size_t)t * p.top_k + i] = i < count ? chosen[i] : -1;
      p.weights[(size_t)t * p.top_k + i] = i < count ? w[i] : 0.0f;
    }
  }
}

hipError_t launch_router(const RouterParams &p, hipStream_t st) {
  const uint32_t n_eg = (p.n_experts + kRouterWaves - 1) / kRouterWaves;
  const uint32_t n_tg = (p.n_tokens + kRouterTokGroup - 1) / kRouterTokGroup;
  const bool vec = p.d_model % 4 == 0 && (uintptr_t)p.gate % 16 == 0 && (uintptr_t)p.x % 16 == 0;
  if (vec) hipLaunchKernelGGL(router_logits_kernel<true>, dim3(n_eg * n_tg), dim3(kRouterThreads), 0, st, p);
  else hipLaunchKernelGGL(router_logits_kernel<false>, dim3(n_eg * n_tg), dim3(kRouterThreads), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds = sizeof(float) * 2 * (size_t)p.n_experts;
  hipLaunchKernelGGL(router_kernel, dim3(p.n_tokens), dim3(kSelThreads), lds, st, p);
  return hipGetLastError();
}

}  // namespace mer
