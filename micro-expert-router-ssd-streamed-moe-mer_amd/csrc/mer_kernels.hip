// mer_kernels.hip -- gfx950 kernels of the routed-expert SwiGLU FFN.
//
// Hot path (reference inference.rs:3291-3306 / :3636-3746, the expert math
// behind engine.rs:1761-1848 and the combine of engine.rs:5548-5639):
//   prep_kernel          x -> block fixed-point digit planes (once per
//                        token); expert id -> blob pointer (once per slot)
//   proj_kernel<FUSED>   h_i = silu(W_gate,i x) * (W_up,i x), written as
//                        digit planes for the down projection
//   proj_kernel<!FUSED>  p_i = W_down,i h_i over column slices
//   combine_kernel       out = [x +] sum_i w_i p_i
//
// Decomposition of proj_kernel.  A workgroup (4 waves) owns one (expert
// instance, column slice, 32-row tile); each wave owns 8 rows of the tile.
// A wave64 is cut into 64/G lane groups of G lanes (G = 16, 32 or 64); a
// lane group owns G*CPL consecutive 64-weight chunks of the slice and walks
// its rows R at a time.  Each weight byte is streamed from HBM exactly once
// with 16-byte loads and consumed by packed integer dot instructions; the
// loads of the next pass are in flight while a pass is computed, and the
// first pass is issued before the input digits are fetched, so no
// prologue latency sits in front of the weight stream.  Row sums are
// reduced across the G lanes with shuffles.  The gate/up kernel packs its
// tile of h = silu(g) * u into digit planes for the down kernel.
#include "mer_internal.hpp"

namespace mer {

__device__ uint32_t g_device_status;

__device__ __forceinline__ void record_status(uint32_t code) {
  atomicCAS(&g_device_status, 0u, code);
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Quantise `nblocks` 32-element blocks of the f32 vector `x` into digit
// planes (dig, 24 dwords per block) and block scales (scale).  All threads
// of the workgroup call this with the same arguments; the kGroups threads
// of one block are adjacent lanes of one wave and share its max by shuffles.
template <int FMT>
__device__ __forceinline__ void pack_vector(const float *x, uint32_t nblocks, uint32_t *dig, float *scale) {
  using D = DigitTraits<FMT>;
  const uint32_t ngroups = nblocks * D::kGroups;
  for (uint32_t base = 0; base < ngroups; base += blockDim.x) {
    const uint32_t g = base + threadIdx.x;
    const bool valid = g < ngroups;
    const uint32_t b = g / D::kGroups, m = g % D::kGroups;
    float v[D::kGroupElems];
    float amax = 0.f;
    int finite = 1;
    if (valid) {
      const float *xb = x + (size_t)b * 32;
      if constexpr (FMT == FMT_Q4_0) {
        const float4 lo = *reinterpret_cast<const float4 *>(xb + 4 * m);
        const float4 hi = *reinterpret_cast<const float4 *>(xb + 16 + 4 * m);
        v[0] = lo.x; v[1] = hi.x; v[2] = lo.y; v[3] = hi.y;
        v[4] = lo.z; v[5] = hi.z; v[6] = lo.w; v[7] = hi.w;
      } else {
        const float4 a = *reinterpret_cast<const float4 *>(xb + 4 * m);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      }
#pragma unroll
      for (int i = 0; i < D::kGroupElems; ++i) {
        amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
        finite &= __builtin_isfinite(v[i]) ? 1 : 0;
      }
    } else {
#pragma unroll
      for (int i = 0; i < D::kGroupElems; ++i) v[i] = 0.f;
    }
#pragma unroll
    for (int off = 1; off < D::kGroups; off <<= 1) {
      amax = __builtin_fmaxf(amax, __shfl_xor(amax, off, 64));
      finite &= __shfl_xor(finite, off, 64);
    }
    if (valid) {
      const BlockScale bs = make_block_scale(amax, finite != 0);
      uint32_t plane[D::kPlanes];
      pack_group<FMT>(v, bs.inv, plane);
#pragma unroll
      for (int k = 0; k < D::kPlanes; ++k) dig[(size_t)b * kBlockDigitDwords + k * D::kGroups + m] = plane[k];
      if (m == 0) scale[b] = bs.s;
    }
  }
}

// One workgroup per token: pack x[t] (fast path only) and resolve the blob
// pointer of each of the token's expert slots.  An id outside the table or
// a non-resident entry resolves to null and records a residency miss,
// except in a zero-weight slot, which the combine skips (engine.rs:5575-5580).
template <int FMT>
__global__ __launch_bounds__(256) void prep_kernel(PrepParams q) {
  const uint32_t t = blockIdx.x;
  if (threadIdx.x < q.top_k) {
    const uint32_t inst = t * q.top_k + threadIdx.x;
    const uint8_t *ptr = q.single;
    if (!ptr) {
      const int32_t id = q.ids[inst];
      const bool unused = q.weights && q.weights[inst] == 0.0f;
      if (id < 0 || (uint32_t)id >= q.table_len) {
        if (!unused) record_status(16u /* MER_ERR_RESIDENCY_MISS */);
      } else {
        ptr = reinterpret_cast<const uint8_t *>(q.table[id]);
        if (!ptr && !unused) record_status(16u);
      }
    }
    q.inst_ptr[inst] = ptr;
  }
  if (q.xq_dig) {
    const size_t b0 = (size_t)t * q.blocks;
    pack_vector<FMT>(q.x + (size_t)t * q.d_model, q.blocks, q.xq_dig + b0 * kBlockDigitDwords, q.xq_scale + b0);
  }
}

template <int FMT, int G, int CPL, int R, bool FUSED>
__global__ __launch_bounds__(256) void proj_kernel(ProjParams p) {
  using T = FmtTraits<FMT>;
  constexpr int kGroups = 64 / G;
  constexpr int kStreams = FUSED ? 2 : 1;
  constexpr uint32_t kStep = R * kGroups;  // rows a wave advances per pass
  static_assert(kRowsPerWave % kStep == 0, "passes must tile the wave's rows");
  __shared__ float s_h[kTileRows];

  const uint32_t per_inst = p.slices * p.tiles;
  const uint32_t inst = blockIdx.x / per_inst;
  const uint32_t rem = blockIdx.x % per_inst;
  const uint32_t slice = rem / p.tiles;
  const uint32_t tile = rem % p.tiles;
  const uint32_t wave = threadIdx.x / 64u;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane / G;
  const uint32_t gl = lane % G;
  const uint32_t tile_r0 = tile * kTileRows;
  const uint32_t r_end = min(p.rows, tile_r0 + (wave + 1) * kRowsPerWave);
  const uint32_t c_begin = slice * p.chunks_per_slice;
  const uint32_t c_count = min(p.chunks_per_slice, p.chunks - c_begin);

  const uint8_t *expert = p.inst_ptr[inst];
  if (!expert) {  // uniform over the workgroup: this tile contributes zeros
    if constexpr (FUSED) {
      const size_t b0 = (size_t)inst * p.hq_blocks + tile_r0 / 32;
      if (threadIdx.x < kBlockDigitDwords) p.hq_dig[b0 * kBlockDigitDwords + threadIdx.x] = 0u;
      if (threadIdx.x == 0) p.hq_scale[b0] = 0.f;
    } else {
      float *out = p.out + ((size_t)inst * p.slices + slice) * p.rows;
      if (threadIdx.x < kTileRows) out[tile_r0 + threadIdx.x] = 0.f;
    }
    return;
  }
  const uint8_t *w0 = expert + p.proj_off0;
  const uint8_t *w1 = expert + p.proj_off1;  // up projection (FUSED only)
  const size_t row_bytes = (size_t)p.chunks * T::kChunkBytes;

  uint32_t lchunk[CPL];
  bool valid[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    lchunk[i] = gl + (uint32_t)i * G;
    valid[i] = lchunk[i] < c_count;
  }

  using WBuf = uint32_t[kStreams][CPL][R][T::kChunkDwords];
  auto load_pass = [&](uint32_t r0, WBuf &wb) {
#pragma unroll
    for (int sidx = 0; sidx < kStreams; ++sidx)
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int j = 0; j < R; ++j) {
          if (valid[i] && r0 + j < r_end) {
            const uint8_t *base = (sidx == 0 ? w0 : w1) + (size_t)(r0 + j) * row_bytes +
                                  (size_t)(c_begin + lchunk[i]) * T::kChunkBytes;
            load_chunk<FMT>(base, wb[sidx][i][j]);
          } else {
#pragma unroll
            for (int k = 0; k < T::kChunkDwords; ++k) wb[sidx][i][j][k] = 0u;
          }
        }
  };

  // input digits of the lane's chunk (its slice of x or h), from global
  const size_t xb0 = (size_t)(inst / p.x_div) * p.xq_blocks + 2 * (size_t)c_begin;
  uint32_t xd[2 * kBlockDigitDwords];
  float xsc[2];
  auto fetch_x = [&](int i) {
    if (valid[i]) {
      const size_t b = xb0 + 2 * (size_t)lchunk[i];
      const uint4 *d4 = reinterpret_cast<const uint4 *>(p.xq_dig + b * kBlockDigitDwords);
#pragma unroll
      for (int k = 0; k < 2 * kBlockDigitDwords / 4; ++k) {
        const uint4 v = d4[k];
        xd[4 * k] = v.x; xd[4 * k + 1] = v.y; xd[4 * k + 2] = v.z; xd[4 * k + 3] = v.w;
      }
      const float2 sc = *reinterpret_cast<const float2 *>(p.xq_scale + b);
      xsc[0] = sc.x;
      xsc[1] = sc.y;
    } else {
#pragma unroll
      for (int k = 0; k < 2 * kBlockDigitDwords; ++k) xd[k] = 0u;
      xsc[0] = xsc[1] = 0.f;
    }
  };

  auto compute_pass = [&](uint32_t r0, WBuf &wb) {
    float acc[kStreams][R];
#pragma unroll
    for (int sidx = 0; sidx < kStreams; ++sidx)
#pragma unroll
      for (int j = 0; j < R; ++j) acc[sidx][j] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if constexpr (CPL > 1) fetch_x(i);
#pragma unroll
      for (int sidx = 0; sidx < kStreams; ++sidx)
#pragma unroll
        for (int j = 0; j < R; ++j) acc[sidx][j] += chunk_idot<FMT>(wb[sidx][i][j], xd, xsc);
    }
#pragma unroll
    for (int sidx = 0; sidx < kStreams; ++sidx)
#pragma unroll
      for (int j = 0; j < R; ++j) acc[sidx][j] = group_sum<G>(acc[sidx][j]);
    if (gl == 0) {
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const uint32_t r = r0 + j;
        if (r < r_end) {
          if constexpr (FUSED) {
            const float h = silu_mul(acc[0][j], acc[1][j], p.swiglu_limit);
            s_h[r - tile_r0] = h;
            if (p.out) p.out[(size_t)inst * p.rows + r] = h;
          } else {
            p.out[((size_t)inst * p.slices + slice) * p.rows + r] = acc[0][j];
          }
        }
      }
    }
  };

  // Software-pipelined walk over the wave's rows: pass n+1's loads are
  // issued before pass n is computed (two register buffers, unrolled by 2).
  uint32_t r0 = tile_r0 + wave * kRowsPerWave + grp * R;
  if (r0 < r_end) {
    WBuf wa, wb;
    load_pass(r0, wa);
    if constexpr (CPL == 1) fetch_x(0);
    while (true) {
      const uint32_t r1 = r0 + kStep;
      if (r1 < r_end) load_pass(r1, wb);
      compute_pass(r0, wa);
      if (r1 >= r_end) break;
      const uint32_t r2 = r1 + kStep;
      if (r2 < r_end) load_pass(r2, wa);
      compute_pass(r1, wb);
      if (r2 >= r_end) break;
      r0 = r2;
    }
  }

  if constexpr (FUSED) {
    // this tile of h -> digit planes for the down projection
    __syncthreads();
    const size_t b0 = (size_t)inst * p.hq_blocks + tile_r0 / 32;
    pack_vector<FMT>(s_h, kTileRows / 32, p.hq_dig + b0 * kBlockDigitDwords, p.hq_scale + b0);
  }
}

// Flat-layout fallback for any shape / alignment: one thread per output
// row, weights decoded element by element in the reference's flat block
// order (q8_0_matvec_scalar_flat, inference.rs:3618-3632).
template <int FMT>
__global__ __launch_bounds__(256) void generic_kernel(GenericParams p) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t inst = t / p.rows;
  if (inst >= p.n_inst) return;
  const uint32_t r = t % p.rows;
  float *out = p.out + (size_t)inst * p.rows;
  const uint8_t *expert = p.inst_ptr[inst];
  if (!expert) {
    out[r] = 0.f;
    return;
  }
  const float *x = p.x + (size_t)(inst / p.x_div) * p.x_stride;
  const uint8_t *g = expert + p.proj_off0;
  const uint8_t *u = expert + p.proj_off1;
  float ag = 0.f, au = 0.f;
  for (uint32_t c = 0; c < p.cols; ++c) {
    const size_t flat = (size_t)r * p.cols + c;
    const float xv = x[c];
    ag = __builtin_fmaf(flat_weight<FMT>(g, flat), xv, ag);
    if (p.fused) au = __builtin_fmaf(flat_weight<FMT>(u, flat), xv, au);
  }
  out[r] = p.fused ? silu_mul(ag, au, p.swiglu_limit) : ag;
}

// out[t][j] = base + sum_i w[t,i] * sum_s partial[t,i,s][j]
// base = x (RESIDUAL), out (ACCUMULATE) or 0.  Slots with w == 0 are
// skipped as in the engine's WeightedInto accumulate (engine.rs:5575-5580).
__global__ __launch_bounds__(256) void combine_kernel(CombineParams c) {
  const size_t t_j = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t_j >= (size_t)c.n_tokens * c.d_model) return;
  const uint32_t t = (uint32_t)(t_j / c.d_model);
  const uint32_t j = (uint32_t)(t_j % c.d_model);
  float acc = 0.f;
  for (uint32_t i = 0; i < c.top_k; ++i) {
    const float w = c.weights ? c.weights[(size_t)t * c.top_k + i] : 1.0f;
    if (c.weights && w == 0.0f) continue;
    const float *pp = c.partial + ((size_t)(t * c.top_k + i) * c.slices) * c.d_model + j;
    float y = pp[0];
    for (uint32_t s = 1; s < c.slices; ++s) y += pp[(size_t)s * c.d_model];
    acc = c.weights ? acc + w * y : acc + y;
  }
  float base = 0.f;
  if (c.flags & 1u) base = c.x[t_j];
  else if (c.flags & 2u) base = c.out[t_j];
  c.out[t_j] = (c.flags & 3u) ? base + acc : acc;
}

// dequantize_*_to_f32: one thread per block; tail block truncated.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *src, size_t n_weights,
                                                      float *dst) {
  const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t nblocks = (n_weights + 31) / 32;
  if (blk >= nblocks) return;
  const uint8_t *b = src + blk * FmtTraits<FMT>::kBlockBytes;
  const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
  const size_t base = blk * 32;
  const size_t n = n_weights - base < 32 ? n_weights - base : 32;
  for (size_t i = 0; i < n; ++i) {
    float v;
    if constexpr (FMT == FMT_Q4_0) {
      const uint8_t byte = b[2 + (i & 15)];
      v = d * (float)((i < 16 ? (byte & 0x0f) : (byte >> 4)) - 8);
    } else {
      v = d * (float)(int8_t)b[2 + i];
    }
    dst[base + i] = v;
  }
}

// Raw Q4_0 qualification matvec: row r reads blocks w_block_off + r*bpr ..
__global__ __launch_bounds__(256) void q4_raw_matvec_kernel(const uint8_t *w, size_t w_block_off,
                                                            uint32_t rows, uint32_t bpr,
                                                            const float *x, float *y) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float sum = 0.f;
  for (uint32_t k = 0; k < bpr; ++k) {
    const uint8_t *b = w + (w_block_off + (size_t)r * bpr + k) * 18;
    const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    for (int c = 0; c < 32; ++c) {
      const uint8_t byte = b[2 + (c & 15)];
      const float wv = d * (float)((c < 16 ? (byte & 0x0f) : (byte >> 4)) - 8);
      sum = __builtin_fmaf(wv, x[k * 32 + c], sum);
    }
  }
  y[r] = sum;
}

// Counter-based synthetic generator; byte-for-byte the oracle's
// mo_bench_fill_q4_0 / mo_bench_fill_q8_0.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <int FMT>
__global__ __launch_bounds__(256) void fill_kernel(uint64_t seed, uint64_t expert, uint64_t block_begin,
                                                   uint64_t n_blocks, float lo, float hi, uint8_t *dst) {
  const uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n_blocks) return;
  const uint64_t key = seed * 0x9E3779B97F4A7C15ull + expert * 0xD1B54A32D192ED03ull + 9 * (block_begin + k);
  const float u = (float)(uint32_t)(mix64(key + 8) >> 40) * (1.0f / 16777216.0f);
  const uint16_t s = f32_to_f16_bits(lo + (hi - lo) * u);
  uint8_t *o = dst + k * FmtTraits<FMT>::kBlockBytes;
  uint16_t *o16 = reinterpret_cast<uint16_t *>(o);  // blocks start 2-byte aligned
  o16[0] = s;
  if constexpr (FMT == FMT_Q4_0) {
    const uint64_t a = mix64(key), b = mix64(key + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o16[1 + i] = (uint16_t)(a >> (16 * i));
      o16[5 + i] = (uint16_t)(b >> (16 * i));
    }
  } else {
#pragma unroll
    for (int wi = 0; wi < 8; ++wi) {
      const uint64_t v = mix64(key + (uint64_t)wi);
      uint8_t q[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const uint32_t v16 = (uint32_t)(v >> (16 * f)) & 0xffffu;
        q[f] = (uint8_t)(int8_t)((int)((v16 * 255u) >> 16) - 127);
      }
      o16[1 + 2 * wi] = (uint16_t)(q[0] | (q[1] << 8));
      o16[2 + 2 * wi] = (uint16_t)(q[2] | (q[3] << 8));
    }
  }
}

// ---------------------------------------------------------------------
// Host-side launchers.

template <int FMT, int G, int CPL, int R, bool FUSED>
static hipError_t launch_proj_t(const ProjParams &p, hipStream_t st) {
  const uint32_t blocks = p.n_inst * p.slices * p.tiles;
  hipLaunchKernelGGL((proj_kernel<FMT, G, CPL, R, FUSED>), dim3(blocks), dim3(256), 0, st, p);
  return hipGetLastError();
}

// R: rows per pass and lane group; G * ... must tile the 8 rows of a wave.
template <int FMT, bool FUSED>
static hipError_t launch_proj_fmt(const ProjParams &p, int G, int CPL, hipStream_t st) {
  if (G == 16) return launch_proj_t<FMT, 16, 1, 2, FUSED>(p, st);
  if (G == 32) return launch_proj_t<FMT, 32, 1, FUSED ? 2 : 4, FUSED>(p, st);
  switch (CPL) {
    case 1: return launch_proj_t<FMT, 64, 1, FUSED ? 2 : 4, FUSED>(p, st);
    case 2: return launch_proj_t<FMT, 64, 2, 1, FUSED>(p, st);
    case 3: return launch_proj_t<FMT, 64, 3, 1, FUSED>(p, st);
    case 4: return launch_proj_t<FMT, 64, 4, 1, FUSED>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_proj(int fmt, bool fused, const ProjPlan &plan, const ProjParams &p, hipStream_t st) {
  if (fmt == FMT_Q4_0)
    return fused ? launch_proj_fmt<FMT_Q4_0, true>(p, plan.G, plan.CPL, st)
                 : launch_proj_fmt<FMT_Q4_0, false>(p, plan.G, plan.CPL, st);
  return fused ? launch_proj_fmt<FMT_Q8_0, true>(p, plan.G, plan.CPL, st)
               : launch_proj_fmt<FMT_Q8_0, false>(p, plan.G, plan.CPL, st);
}

hipError_t launch_prep(int fmt, const PrepParams &q, uint32_t n_tokens, hipStream_t st) {
  if (fmt == FMT_Q4_0) hipLaunchKernelGGL(prep_kernel<FMT_Q4_0>, dim3(n_tokens), dim3(256), 0, st, q);
  else hipLaunchKernelGGL(prep_kernel<FMT_Q8_0>, dim3(n_tokens), dim3(256), 0, st, q);
  return hipGetLastError();
}

hipError_t launch_generic(int fmt, const GenericParams &p, hipStream_t st) {
  const uint64_t threads = (uint64_t)p.n_inst * p.rows;
  const uint32_t blocks = (uint32_t)((threads + 255) / 256);
  if (blocks == 0) return hipSuccess;
  if (fmt == FMT_Q4_0) hipLaunchKernelGGL(generic_kernel<FMT_Q4_0>, dim3(blocks), dim3(256), 0, st, p);
  else hipLaunchKernelGGL(generic_kernel<FMT_Q8_0>, dim3(blocks), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_combine(const CombineParams &c, hipStream_t st) {
  const uint64_t n = (uint64_t)c.n_tokens * c.d_model;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, c);
  return hipGetLastError();
}

hipError_t launch_dequant(int fmt, const uint8_t *src, size_t n_weights, float *dst, hipStream_t st) {
  const size_t nblocks = (n_weights + 31) / 32;
  if (nblocks == 0) return hipSuccess;
  const uint32_t grid = (uint32_t)((nblocks + 255) / 256);
  if (fmt == FMT_Q4_0) hipLaunchKernelGGL(dequant_kernel<FMT_Q4_0>, dim3(grid), dim3(256), 0, st, src, n_weights, dst);
  else hipLaunchKernelGGL(dequant_kernel<FMT_Q8_0>, dim3(grid), dim3(256), 0, st, src, n_weights, dst);
  return hipGetLastError();
}

hipError_t launch_q4_raw(const uint8_t *w, size_t w_block_off, uint32_t rows, uint32_t bpr,
                         const float *x, float *y, hipStream_t st) {
  hipLaunchKernelGGL(q4_raw_matvec_kernel, dim3((rows + 255) / 256), dim3(256), 0, st, w, w_block_off,
                     rows, bpr, x, y);
  return hipGetLastError();
}

hipError_t launch_fill(int fmt, uint64_t seed, uint64_t expert, uint64_t block_begin, uint64_t n_blocks,
                       float lo, float hi, uint8_t *dst, hipStream_t st) {
  if (n_blocks == 0) return hipSuccess;
  const uint64_t grid = (n_blocks + 255) / 256;
  // keep each launch within a 32-bit grid
  const uint64_t max_grid = 1ull << 30;
  for (uint64_t g0 = 0; g0 < grid; g0 += max_grid) {
    const uint64_t g = grid - g0 < max_grid ? grid - g0 : max_grid;
    const uint64_t b0 = g0 * 256;
    const uint64_t nb = n_blocks - b0 < g * 256 ? n_blocks - b0 : g * 256;
    uint8_t *d = dst + b0 * (fmt == FMT_Q4_0 ? 18 : 34);
    if (fmt == FMT_Q4_0)
      hipLaunchKernelGGL(fill_kernel<FMT_Q4_0>, dim3((uint32_t)g), dim3(256), 0, st, seed, expert,
                         block_begin + b0, nb, lo, hi, d);
    else
      hipLaunchKernelGGL(fill_kernel<FMT_Q8_0>, dim3((uint32_t)g), dim3(256), 0, st, seed, expert,
                         block_begin + b0, nb, lo, hi, d);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// f16 <-> f32 staging of the f16-view entry point: x [d_model] repeated
// n_rep times, and the outputs rounded to f16 (round to nearest even).
__global__ __launch_bounds__(256) void f16_in_kernel(const _Float16 *x, size_t d_model, size_t n_rep, float *dst) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= d_model * n_rep) return;
  dst[i] = (float)x[i % d_model];
}
__global__ __launch_bounds__(256) void f16_out_kernel(const float *src, size_t n, _Float16 *dst) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = (_Float16)src[i];
}

hipError_t launch_f16_in(const uint16_t *x, size_t d_model, size_t n_rep, float *dst, hipStream_t st) {
  const size_t n = d_model * n_rep;
  hipLaunchKernelGGL(f16_in_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const _Float16 *>(x), d_model, n_rep, dst);
  return hipGetLastError();
}
hipError_t launch_f16_out(const float *src, size_t n, uint16_t *dst, hipStream_t st) {
  hipLaunchKernelGGL(f16_out_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, src, n,
                     reinterpret_cast<_Float16 *>(dst));
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void zero_kernel(float *dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = 0.f;
}

hipError_t launch_zero(float *dst, size_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, dst, n);
  return hipGetLastError();
}

uint32_t *device_status_ptr() {
  void *ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_device_status)) != hipSuccess) return nullptr;
  return reinterpret_cast<uint32_t *>(ptr);
}

hipError_t read_and_clear_device_status(uint32_t *out) {
  uint32_t zero = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_device_status), sizeof(uint32_t), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return e;
  return hipMemcpyToSymbol(HIP_SYMBOL(g_device_status), &zero, sizeof(uint32_t), 0, hipMemcpyHostToDevice);
}

}  // namespace mer
