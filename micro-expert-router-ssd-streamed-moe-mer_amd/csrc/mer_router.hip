// mer_router.hip -- LinearGate routing on the GPU for gfx950.
//
// One 256-thread workgroup per token restates LinearGate::route_with_scratch
// (gating.rs:395-476) with its full routing surface (with_routing,
// gating.rs:207-268):
//   logits    = W x                               (W: [n_experts][d_model] f32)
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

}  // namespace

__global__ __launch_bounds__(kRouterThreads) void router_kernel(RouterParams p) {
  extern __shared__ float smem[];
  float *scores = smem;                               // [n_experts]
  float *selection = scores + p.n_experts;            // [n_experts]
  __shared__ float red_f[kRouterWaves];
  __shared__ int32_t red_k[kRouterWaves], red_i[kRouterWaves];
  __shared__ uint32_t group_ok[kMaxRouterExperts / 32];
  __shared__ int32_t chosen[kMaxRouterTopK];
  __shared__ int32_t flag_bad;

  const uint32_t t = blockIdx.x;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const float *x = p.x + (size_t)t * p.d_model;  // read by every wave: stays in L1/L2
  if (tid == 0) flag_bad = 0;
  __syncthreads();

  // ---- logits = W x: one expert per wave at a time ----------------------
  for (uint32_t e = wave; e < p.n_experts; e += kRouterWaves) {
    const float *w = p.gate + (size_t)e * p.d_model;
    float acc = 0.f;
    for (uint32_t d = lane; d < p.d_model; d += 64) acc = __builtin_fmaf(w[d], x[d], acc);
    acc = wave_sum(acc);
    if (lane == 0) scores[e] = acc;
  }
  __syncthreads();
  if (p.logits)
    for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads) p.logits[(size_t)t * p.n_experts + e] = scores[e];

  // ---- scores -------------------------------------------------------------
  if (p.scoring == 0) {
    // softmax: max over non-NaN values; a NaN or a non-finite max makes the
    // row uniform (softmax_inplace's fallback)
    float m = -INFINITY;
    for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads) {
      const float v = scores[e];
      if (v != v) flag_bad = 1;  // benign race: every writer stores 1
      else m = __builtin_fmaxf(m, v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = red_f[0];
    for (int i = 1; i < kRouterWaves; ++i) m = __builtin_fmaxf(m, red_f[i]);
    const bool uniform = flag_bad || !__builtin_isfinite(m);
    __syncthreads();
    float s = 0.f;
    for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads) {
      const float v = uniform ? 1.f : expf(scores[e] - m);
      scores[e] = v;
      s += v;
    }
    s = wave_sum(s);
    if (lane == 0) red_f[wave] = s;
    __syncthreads();
    float sum = 0.f;
    for (int i = 0; i < kRouterWaves; ++i) sum += red_f[i];
    for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads)
      scores[e] = uniform ? 1.0f / (float)p.n_experts : (sum > 0.f ? scores[e] / sum : scores[e]);
  } else {
    for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads) scores[e] = 1.0f / (1.0f + expf(-scores[e]));
  }
  __syncthreads();
  for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads)
    selection[e] = p.bias ? scores[e] + p.bias[e] : scores[e];
  for (uint32_t i = tid; i < kMaxRouterExperts / 32; i += kRouterThreads) group_ok[i] = 0xffffffffu;
  __syncthreads();

  // ---- optional group filter ----------------------------------------------
  const bool grouped = p.n_group > 1 && p.topk_group > 0 && p.topk_group < p.n_group && p.n_experts % p.n_group == 0;
  if (grouped && tid == 0) {
    const uint32_t gs = p.n_experts / p.n_group;
    int32_t sel_g[kMaxRouterGroups];  // surviving groups, best first
    float sel_s[kMaxRouterGroups];
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

  // ---- top-k: k rounds of a workgroup arg-max ----------------------------
  uint32_t count = 0;
  for (uint32_t r = 0; r < p.top_k; ++r) {
    int32_t bk = INT32_MIN, bi = -1;
    for (uint32_t e = tid; e < p.n_experts; e += kRouterThreads) {
      const float v = selection[e];
      if (!__builtin_isfinite(v) || !((group_ok[e >> 5] >> (e & 31u)) & 1u)) continue;
      bool taken = false;
      for (uint32_t q = 0; q < r; ++q) taken |= chosen[q] == (int32_t)e;
      if (taken) continue;
      const int32_t k = total_key(v);
      if (bi < 0 || better(k, (int32_t)e, bk, bi)) {
        bk = k;
        bi = (int32_t)e;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int32_t ok = __shfl_xor(bk, off, 64), oi = __shfl_xor(bi, off, 64);
      if (oi >= 0 && (bi < 0 || better(ok, oi, bk, bi))) {
        bk = ok;
        bi = oi;
      }
    }
    if (lane == 0) {
      red_k[wave] = bk;
      red_i[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      int32_t k0 = red_k[0], i0 = red_i[0];
      for (int w = 1; w < kRouterWaves; ++w)
        if (red_i[w] >= 0 && (i0 < 0 || better(red_k[w], red_i[w], k0, i0))) {
          k0 = red_k[w];
          i0 = red_i[w];
        }
      chosen[r] = i0;
    }
    __syncthreads();
    if (chosen[r] < 0) break;
    count = r + 1;
  }

  // ---- weights ------------------------------------------------------------
  if (tid == 0) {
    float w[kMaxRouterTopK];
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
  const size_t lds = sizeof(float) * 2 * (size_t)p.n_experts;
  hipLaunchKernelGGL(router_kernel, dim3(p.n_tokens), dim3(kRouterThreads), lds, st, p);
  return hipGetLastError();
}

}  // namespace mer
