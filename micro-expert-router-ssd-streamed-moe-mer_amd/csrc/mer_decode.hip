// mer_decode.hip -- persistent routed-expert decode kernel for gfx950.
//
// One launch runs every MoE layer of a decode step (reference: the
// WeightedInto loop of moe_step_inner, engine.rs:5548-5639, over the expert
// math of inference.rs:3291-3306 / :3636-3746).  A fixed grid of resident
// one-wave workgroups walks a global list of work items, layer by layer:
//   R  resolve the blob pointer of a token's expert slots (ids -> table)
//   P  quantise 16 (Q4_0) / 8 (Q8_0) blocks of a token's layer input into
//      digit planes
//   G  gate/up of one (slot, column slice, 32-row tile): streams the tile's
//      gate and up rows; with one slice it applies SiLU and packs the tile
//      of h into digit planes, otherwise the last slice to arrive does
//   D  down of one (slot, column slice, 32-row tile) -> partial sums; the
//      last (slot, slice) to arrive for a (token, tile) combines
//      out = [x +] sum_i w_i y_i for the tile (combine_outputs_into order)
// Dependencies are counters in global memory: a producer releases its
// stores (agent-scope fence) and increments; a consumer polls, then
// acquires.  Items only wait on items earlier in the list, and the grid
// never exceeds what is co-resident, so the walk always drains; every poll
// is bounded by a wall-clock timeout that records a device status instead
// of hanging.  Waves issue the weight loads of their next item's first two
// passes before waiting on its inputs, so weight streaming overlaps the
// dependency chain between phases and layers.  The last wave to exit
// zeroes the counters for the next launch.
#include "mer_internal.hpp"

namespace mer {

namespace {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

__device__ __forceinline__ uint32_t poll(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
__device__ __forceinline__ void release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }

__device__ __forceinline__ void set_status(const DecodeParams &p, uint32_t code) {
  atomicCAS(p.status, 0u, code);
}

// Wait until *ctr >= target (lane 0 polls), then acquire.  Returns false
// after a timeout: the status is recorded and the launch's abort flag set,
// which makes every later wait return at once, so the grid drains.
__device__ bool wait_for(const DecodeParams &p, const uint32_t *ctr, uint32_t target) {
  uint32_t ok = 1;
  if (lane_id() == 0 && poll(ctr) < target) {
    const uint64_t t0 = wall_clock64();
    while (poll(ctr) < target) {
      if (poll(p.abort_flag) != 0u) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
      if (wall_clock64() - t0 > p.timeout_ticks) {
        set_status(p, 24u /* MER_ERR_RUNTIME_INVARIANT: dependency timeout */);
        __hip_atomic_store(p.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
    }
  }
  ok = __shfl(ok, 0, 64);
  acquire();
  return ok != 0;
}

// Release this wave's stores, then count one arrival.
__device__ __forceinline__ void signal(uint32_t *ctr) {
  release();
  if (lane_id() == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Release, count one arrival, and report whether this was the last of
// `expected` (then acquire the other arrivals' stores).
__device__ __forceinline__ bool arrive_last(uint32_t *ctr, uint32_t expected) {
  release();
  uint32_t old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  const bool last = old + 1 == expected;
  if (last) acquire();
  return last;
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Quantise `nblocks` (<= 64 / groups) blocks of x into digit planes; one
// wave, lane = group.
template <int FMT>
__device__ __forceinline__ void pack_blocks(const float *x, uint32_t nblocks, uint32_t *dig, float *scale) {
  using D = DigitTraits<FMT>;
  const uint32_t g = lane_id();
  const bool valid = g < nblocks * D::kGroups;
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

// Streaming walk of one 32-row tile: lane groups of G lanes, R rows per
// pass, S weight streams (2 = gate and up).  `emit(row, acc[S])` receives
// each row's sums (called on all lanes of the owning group).
template <int FMT, int G, int R, int S>
struct TileWalk {
  using T = FmtTraits<FMT>;
  static constexpr int kGroups = 64 / G;
  static constexpr uint32_t kStep = R * kGroups;
  static constexpr uint32_t kPasses = kTileRows / kStep;
  static_assert(kTileRows % kStep == 0 && kPasses % 2 == 0, "passes must tile 32 rows in pairs");
  using WBuf = uint32_t[S][R][T::kChunkDwords];

  const uint8_t *w[S];
  size_t row_bytes;
  uint32_t r_base;  // first row of this lane group's first pass
  bool valid;       // lane owns a chunk of the slice

  __device__ __forceinline__ void load(uint32_t pass, WBuf &wb) const {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < R; ++j) {
        if (valid) {
          load_chunk<FMT>(w[s] + (size_t)(r_base + pass * kStep + j) * row_bytes, wb[s][j]);
        } else {
#pragma unroll
          for (int k = 0; k < T::kChunkDwords; ++k) wb[s][j][k] = 0u;
        }
      }
  }

  template <class Emit>
  __device__ __forceinline__ void compute(uint32_t pass, WBuf &wb, const uint32_t *xd, const float *xsc,
                                          Emit &&emit) const {
    float acc[S][R];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < R; ++j) acc[s][j] = group_sum<G>(chunk_idot<FMT>(wb[s][j], xd, xsc));
#pragma unroll
    for (int j = 0; j < R; ++j) {
      float a[S];
#pragma unroll
      for (int s = 0; s < S; ++s) a[s] = acc[s][j];
      emit(r_base + pass * kStep + j, a);
    }
  }
};

// Fetch the 48 digit dwords and 2 scales of chunk `c` of a packed vector.
__device__ __forceinline__ void fetch_digits(const uint32_t *dig, const float *sc, size_t block0, bool valid,
                                             uint32_t (&xd)[2 * kBlockDigitDwords], float (&xsc)[2]) {
  if (valid) {
    const uint4 *d4 = reinterpret_cast<const uint4 *>(dig + block0 * kBlockDigitDwords);
#pragma unroll
    for (int k = 0; k < 2 * kBlockDigitDwords / 4; ++k) {
      const uint4 v = d4[k];
      xd[4 * k] = v.x; xd[4 * k + 1] = v.y; xd[4 * k + 2] = v.z; xd[4 * k + 3] = v.w;
    }
    const float2 s2 = *reinterpret_cast<const float2 *>(sc + block0);
    xsc[0] = s2.x;
    xsc[1] = s2.y;
  } else {
#pragma unroll
    for (int k = 0; k < 2 * kBlockDigitDwords; ++k) xd[k] = 0u;
    xsc[0] = xsc[1] = 0.f;
  }
}

}  // namespace

template <int FMT, int GG, int GD>
__global__ __launch_bounds__(64) void decode_kernel(DecodeParams p) {
  __shared__ float s_h[kTileRows];
  const uint32_t lane = lane_id();
  using D = DigitTraits<FMT>;
  constexpr uint32_t kPackBlocks = 64 / D::kGroups;

  for (uint64_t gi = blockIdx.x; gi < p.total_items; gi += gridDim.x) {
    const uint32_t l = (uint32_t)(gi / p.items_per_layer);
    const uint32_t j = (uint32_t)(gi % p.items_per_layer);
    const LayerArgs &la = p.layers[l];
    uint32_t *cnt = p.counters + (size_t)l * p.cnt_per_layer;
    const uint8_t **inst_ptr = p.inst_ptr + (size_t)l * p.n_inst;
    uint32_t *xq_dig = p.xq_dig + (size_t)l * p.n_tok * p.xblocks * kBlockDigitDwords;
    float *xq_scale = p.xq_scale + (size_t)l * p.n_tok * p.xblocks;
    uint32_t *hq_dig = p.hq_dig + (size_t)l * p.n_inst * p.hblocks * kBlockDigitDwords;
    float *hq_scale = p.hq_scale + (size_t)l * p.n_inst * p.hblocks;
    // layer input of token t
    const float *xsrc = (p.flags & kFlagChain) && l > 0 ? p.layers[l - 1].out : la.x;

    if (j < p.off_p) {
      // ---- R: resolve the token's expert slots ----------------------------
      const uint32_t t = j;
      if (lane < p.top_k) {
        const uint32_t inst = t * p.top_k + lane;
        const uint8_t *ptr = p.single;
        if (!ptr) {
          const int32_t id = la.ids[inst];
          if (id < 0 || (uint32_t)id >= la.table_len) {
            set_status(p, 16u /* MER_ERR_RESIDENCY_MISS */);
          } else {
            ptr = reinterpret_cast<const uint8_t *>(la.table[id]);
            if (!ptr) set_status(p, 16u);
          }
        }
        inst_ptr[inst] = ptr;
      }
      signal(cnt + p.c_r + t);
    } else if (j < p.off_g) {
      // ---- P: pack part of the token's layer input ------------------------
      const uint32_t idx = j - p.off_p;
      const uint32_t t = idx / p.p_items;
      const uint32_t part = idx % p.p_items;
      if (l > 0) {  // layers run in order: layer l reads after layer l-1 wrote
        const uint32_t *prev = p.counters + (size_t)(l - 1) * p.cnt_per_layer + p.c_c;
        wait_for(p, prev + t, p.d_tiles);
      }
      const uint32_t b0 = part * kPackBlocks;
      const uint32_t nb = min(kPackBlocks, p.xblocks - b0);
      const size_t tb = (size_t)t * p.xblocks + b0;
      pack_blocks<FMT>(xsrc + (size_t)t * p.d_model + (size_t)b0 * 32, nb, xq_dig + tb * kBlockDigitDwords,
                       xq_scale + tb);
      signal(cnt + p.c_p + t);
    } else if (j < p.off_d) {
      // ---- G: gate/up of one (slot, column slice, tile) -------------------
      const uint32_t idx = j - p.off_g;
      const uint32_t per_inst = p.g_tiles * p.g_slices;
      const uint32_t inst = idx / per_inst;
      const uint32_t tile = (idx % per_inst) / p.g_slices;
      const uint32_t gs = idx % p.g_slices;
      const uint32_t t = inst / p.top_k;
      wait_for(p, cnt + p.c_r + t, 1);
      const uint8_t *expert = inst_ptr[inst];
      const uint32_t dslice = tile * 32 / (p.d_cps * 64);
      using W = TileWalk<FMT, GG, 2, 2>;
      const uint32_t grp = lane / GG, gl = lane % GG;
      const uint32_t c_begin = gs * p.g_cps;
      const uint32_t c = c_begin + gl;
      W walk;
      walk.valid = expert && gl < p.g_cps && c < p.g_chunks;
      walk.row_bytes = (size_t)p.g_chunks * FmtTraits<FMT>::kChunkBytes;
      walk.w[0] = expert + (size_t)c * FmtTraits<FMT>::kChunkBytes;
      walk.w[1] = walk.w[0] + p.proj_bytes;
      walk.r_base = tile * kTileRows + grp * 2;
      typename W::WBuf wa, wb;
      walk.load(0, wa);
      walk.load(1, wb);
      wait_for(p, cnt + p.c_p + t, p.p_items);
      uint32_t xd[2 * kBlockDigitDwords];
      float xsc[2];
      fetch_digits(xq_dig, xq_scale, (size_t)t * p.xblocks + 2 * (size_t)c, walk.valid, xd, xsc);
      float *gpart = p.gpart + (((size_t)l * p.n_inst + inst) * p.g_slices + gs) * 2 * p.d_ff;
      const bool single_slice = p.g_slices == 1;
      auto emit = [&](uint32_t r, const float (&a)[2]) {
        if (gl == 0) {
          if (single_slice) {
            s_h[r - tile * kTileRows] = expert ? silu_mul(a[0], a[1]) : 0.f;
          } else {
            gpart[r] = a[0];
            gpart[p.d_ff + r] = a[1];
          }
        }
      };
#pragma unroll 1
      for (uint32_t pass = 0; pass < W::kPasses; pass += 2) {
        walk.compute(pass, wa, xd, xsc, emit);
        if (pass + 2 < W::kPasses) walk.load(pass + 2, wa);
        walk.compute(pass + 1, wb, xd, xsc, emit);
        if (pass + 3 < W::kPasses) walk.load(pass + 3, wb);
      }
      bool pack = single_slice;
      if (!single_slice) {
        pack = arrive_last(cnt + p.c_ga + (size_t)inst * p.g_tiles + tile, p.g_slices);
        if (pack && lane < kTileRows) {
          const size_t base = ((size_t)l * p.n_inst + inst) * p.g_slices * 2 * p.d_ff;
          const uint32_t r = tile * kTileRows + lane;
          float g = 0.f, u = 0.f;
          for (uint32_t s = 0; s < p.g_slices; ++s) {
            g += p.gpart[base + (size_t)s * 2 * p.d_ff + r];
            u += p.gpart[base + (size_t)s * 2 * p.d_ff + p.d_ff + r];
          }
          s_h[lane] = silu_mul(g, u);
        }
      }
      if (pack) {
        __syncthreads();
        const size_t hb = (size_t)inst * p.hblocks + tile;
        pack_blocks<FMT>(s_h, 1, hq_dig + hb * kBlockDigitDwords, hq_scale + hb);
        signal(cnt + p.c_gd + (size_t)inst * p.d_slices + dslice);
      }
    } else {
      // ---- D: down of one (slot, column slice, tile) + combine -------------
      const uint32_t idx = j - p.off_d;
      const uint32_t per_tok = p.d_tiles * p.top_k * p.d_slices;
      const uint32_t t = idx / per_tok;
      const uint32_t rem = idx % per_tok;
      const uint32_t tile = rem / (p.top_k * p.d_slices);
      const uint32_t slot = (rem / p.d_slices) % p.top_k;
      const uint32_t ds = rem % p.d_slices;
      const uint32_t inst = t * p.top_k + slot;
      wait_for(p, cnt + p.c_r + t, 1);
      const uint8_t *expert = inst_ptr[inst];
      using W = TileWalk<FMT, GD, (GD == 16 ? 2 : 4), 1>;
      const uint32_t grp = lane / GD, gl = lane % GD;
      const uint32_t c = ds * p.d_cps + gl;
      W walk;
      walk.valid = expert && gl < p.d_cps && c < p.d_chunks;
      walk.row_bytes = (size_t)p.d_chunks * FmtTraits<FMT>::kChunkBytes;
      walk.w[0] = expert + 2 * p.proj_bytes + (size_t)c * FmtTraits<FMT>::kChunkBytes;
      walk.r_base = tile * kTileRows + grp * (GD == 16 ? 2 : 4);
      typename W::WBuf wa, wb;
      walk.load(0, wa);
      walk.load(1, wb);
      // the h planes of this column slice
      const uint32_t first_tile = ds * p.d_cps * 2;
      const uint32_t n_tiles = min(p.d_cps * 2, p.g_tiles - first_tile);
      wait_for(p, cnt + p.c_gd + (size_t)inst * p.d_slices + ds, n_tiles);
      uint32_t xd[2 * kBlockDigitDwords];
      float xsc[2];
      fetch_digits(hq_dig, hq_scale, (size_t)inst * p.hblocks + 2 * (size_t)c, walk.valid, xd, xsc);
      float *part = p.partial + (((size_t)l * p.n_inst + inst) * p.d_slices + ds) * p.d_model;
      auto emit = [&](uint32_t r, const float (&a)[1]) {
        if (gl == 0) part[r] = a[0];
      };
#pragma unroll 1
      for (uint32_t pass = 0; pass < W::kPasses; pass += 2) {
        walk.compute(pass, wa, xd, xsc, emit);
        if (pass + 2 < W::kPasses) walk.load(pass + 2, wa);
        walk.compute(pass + 1, wb, xd, xsc, emit);
        if (pass + 3 < W::kPasses) walk.load(pass + 3, wb);
      }
      if (arrive_last(cnt + p.c_da + (size_t)t * p.d_tiles + tile, p.top_k * p.d_slices)) {
        // combine_outputs_into order: acc = 0; acc += w_i * y_i by slot;
        // zero-weight slots skipped as in the engine (engine.rs:5575-5580)
        if (lane < kTileRows) {
          const uint32_t r = tile * kTileRows + lane;
          float acc = 0.f;
          for (uint32_t i = 0; i < p.top_k; ++i) {
            const float w = la.weights ? la.weights[t * p.top_k + i] : 1.0f;
            if (la.weights && w == 0.0f) continue;
            const float *pp =
                p.partial + (((size_t)l * p.n_inst + t * p.top_k + i) * p.d_slices) * p.d_model + r;
            float y = pp[0];
            for (uint32_t s = 1; s < p.d_slices; ++s) y += pp[(size_t)s * p.d_model];
            acc = la.weights ? acc + w * y : acc + y;
          }
          float *o = la.out + (size_t)t * p.d_model + r;
          if (p.flags & kFlagResidual) *o = xsrc[(size_t)t * p.d_model + r] + acc;
          else if (p.flags & kFlagAccumulate) *o = *o + acc;
          else *o = acc;
        }
        signal(cnt + p.c_c + t);
      }
    }
  }

  // the last wave out zeroes the counters for the next launch
  release();
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(p.exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  if (old + 1 == gridDim.x) {
    acquire();
    for (uint32_t i = lane; i < p.n_counters; i += 64) p.counters[i] = 0u;
    if (lane == 0) {
      *p.abort_flag = 0u;
      *p.exit_count = 0u;
    }
    release();
  }
}

template <int FMT, int GG, int GD>
static const void *decode_fn() {
  return reinterpret_cast<const void *>(&decode_kernel<FMT, GG, GD>);
}

template <int FMT, int GG>
static const void *decode_fn_gd(int gd) {
  if (gd == 16) return decode_fn<FMT, GG, 16>();
  if (gd == 32) return decode_fn<FMT, GG, 32>();
  return decode_fn<FMT, GG, 64>();
}

template <int FMT>
static const void *decode_fn_fmt(int gg, int gd) {
  if (gg == 16) return decode_fn_gd<FMT, 16>(gd);
  if (gg == 32) return decode_fn_gd<FMT, 32>(gd);
  return decode_fn_gd<FMT, 64>(gd);
}

const void *decode_kernel_fn(int fmt, int gg, int gd) {
  return fmt == FMT_Q4_0 ? decode_fn_fmt<FMT_Q4_0>(gg, gd) : decode_fn_fmt<FMT_Q8_0>(gg, gd);
}

hipError_t launch_decode(const void *fn, uint32_t grid, const DecodeParams &p, hipStream_t st) {
  void *args[] = {const_cast<DecodeParams *>(&p)};
  return hipLaunchKernel(fn, dim3(grid), dim3(64), args, 0, st);
}

}  // namespace mer
