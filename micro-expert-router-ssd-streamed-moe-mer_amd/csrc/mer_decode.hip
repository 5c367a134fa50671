// mer_decode.hip -- persistent routed-expert decode kernel for gfx950.
//
// One launch runs every MoE layer of a decode step (reference: the
// WeightedInto loop of moe_step_inner, engine.rs:5548-5639, over the expert
// math of inference.rs:3291-3306 / :3636-3746).  A fixed grid of resident
// one-wave workgroups walks a global list of work items, layer by layer:
//   R  check a token's expert slots (ids -> table) and report residency
//      misses; G and D items look their blob up themselves
//   P  quantise 16 (Q4_0) / 8 (Q8_0) blocks of a token's layer-0 input into
//      digit planes (idle in later layers: their input blocks are packed by
//      the combines of the layer before)
//   G  gate/up of one (slot, column slice, 32-row tile): streams the tile's
//      gate and up rows; with one slice it applies SiLU and packs the tile
//      of h into digit planes, otherwise the last slice to arrive does
//   D  down of one (slot, column slice, 32-row tile) -> partial sums; the
//      last (slot, slice) to arrive for a (token, tile) combines
//      out = [x +] sum_i w_i y_i for the tile (combine_outputs_into order)
//      and packs the same 32 elements of the next layer's input (that
//      output when chained, else the caller's next x) into digit planes;
//      the last combine of a layer sets the layer's release flags, which
//      the next layer's items poll (each on one of 16 lines, so hundreds of
//      waiters do not all poll the line the combines count on); likewise the
//      last h tile of a column slice releases the slice's D items when the
//      number of slices is small
// Dependencies are counters in global memory.  Partial sums and outputs
// handed from one wave to another are written and read with device-scope
// (sc1) accesses, which are coherent across the XCDs for exactly the lines
// they touch.  Digit planes are written with device-scope stores and read
// with ordinary cached loads, so each XCD's L2 serves the many waves that
// read the same vector; every digit line carries the epoch of the launch
// that wrote it, and a reader that finds an older epoch (a copy cached by
// an earlier launch) reads the line again with device-scope loads.  A
// producer drains its stores (s_waitcnt vmcnt(0)) and then increments the
// counter with a device-scope atomic; a consumer polls the counter before
// reading.  No cache-wide writeback or invalidate is ever issued.  Items
// only wait on items earlier in the list, and the grid never exceeds what
// is co-resident, so the walk always drains; every poll is bounded by a
// wall-clock timeout that records a device status instead of hanging.
// Waves issue the weight loads of their next item's first passes before
// waiting on its inputs, so weight streaming overlaps the dependency chain
// between phases and layers.  The last wave to exit zeroes the counters for
// the next launch.
#include <type_traits>

#include "mer_internal.hpp"

namespace mer {

// Source of the epochs the decode launches hand to their successors.
__device__ unsigned long long g_epoch_seq;

namespace {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

__device__ __forceinline__ uint32_t poll(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-scope (sc1) loads and stores for data exchanged between waves.
template <class T>
__device__ __forceinline__ T ld_dev(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void st_dev(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Blob of expert instance `inst` of layer `la` (the same on every lane), or
// null for a residency miss.  Read from the caller's routing arrays, which
// were written before this launch, so ordinary loads see them.
__device__ __forceinline__ const uint8_t *resolve_expert(const DecodeParams &p, const LayerArgs &la, uint32_t inst) {
  if (p.single) return p.single;
  const int32_t id = __builtin_amdgcn_readfirstlane(la.ids[inst]);
  if (id < 0 || (uint32_t)id >= la.table_len) return nullptr;
  const uint64_t v = reinterpret_cast<const uint64_t *>(la.table)[id];
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t *>(join_u32(hi, lo));
}

// Wait for this wave's outstanding stores; keeps the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void drain_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }
// LDS written by some lanes of this wave, read by others: wait for the
// wave's LDS accesses (a wave's LDS instructions complete in order).
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ void set_status(const DecodeParams &p, uint32_t code) {
  atomicCAS(p.status, 0u, code);
}

// Wave priority on the SIMD.  A wave runs its hand-off work (digit
// fetches, arrivals, combines, packing) at raised priority, so the
// instructions on the layer's critical path issue ahead of the weight walks
// of the other waves sharing its SIMD (measured, Mixtral decode: 708 -> 720
// tokens/s; raising the prefetch issue or the walk itself gains nothing).
__device__ __forceinline__ void prio_hi() { __builtin_amdgcn_s_setprio(2); }
__device__ __forceinline__ void prio_lo() { __builtin_amdgcn_s_setprio(0); }

constexpr uint32_t kNapCounter = 16;  // longest nap between polls of a shared counter, in ~0.05 us
constexpr uint32_t kNapFlag = 2;      // ... of a release flag

// Wait until *ctr >= target (lane 0 polls), then acquire.  Returns false
// after a timeout: the status is recorded and the launch's abort flag set,
// which makes every later wait return at once, so the grid drains.
__device__ bool wait_for(const DecodeParams &p, const uint32_t *ctr, uint32_t target, uint32_t max_nap) {
  uint32_t ok = 1;
  if (lane_id() == 0 && poll(ctr) < target) {
    // Exponential backoff from ~0.05 us up to max_nap x ~0.05 us between
    // polls.  Counters that hundreds of waves wait on take long naps
    // (kNapCounter): polling them at full rate floods the memory channel
    // that holds them and slows both their arrivals and the weight streams.
    // Release flags spread their waiters over kReleaseFan lines, so their
    // naps stay short (kNapFlag), which cuts the wake-up latency of every
    // hand-off (measured, Qwen3 decode: ~0.8 us naps 1,108 tokens/s,
    // ~0.1 us naps 1,132).
    const uint64_t t0 = wall_clock64();
    uint32_t nap = 1, n = 0;
    while (poll(ctr) < target) {
      for (uint32_t i = 0; i < nap; ++i) __builtin_amdgcn_s_sleep(2);
      if (nap < max_nap) nap <<= 1;
      if ((++n & 15u) == 0u) {
        if (poll(p.abort_flag) != 0u) {
          ok = 0;
          break;
        }
        if (wall_clock64() - t0 > p.timeout_ticks) {
          set_status(p, 24u /* MER_ERR_RUNTIME_INVARIANT: dependency timeout */);
          __hip_atomic_store(p.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
      }
    }
  }
  ok = __shfl(ok, 0, 64);
  compiler_fence();
  return ok != 0;
}

// Wait until the release flag *flag holds this launch's epoch (lane 0
// polls), then acquire.  Flags are compared for equality: a flag left by any
// other launch holds another epoch and reads as not set.  Timeout and abort
// as wait_for.
__device__ bool wait_flag(const DecodeParams &p, const uint64_t *flag, uint64_t epoch, uint32_t max_nap) {
  uint32_t ok = 1;
  if (lane_id() == 0 && ld_dev(flag) != epoch) {
    const uint64_t t0 = wall_clock64();
    uint32_t nap = 1, n = 0;
    while (ld_dev(flag) != epoch) {
      for (uint32_t i = 0; i < nap; ++i) __builtin_amdgcn_s_sleep(2);
      if (nap < max_nap) nap <<= 1;
      if ((++n & 15u) == 0u) {
        if (poll(p.abort_flag) != 0u) {
          ok = 0;
          break;
        }
        if (wall_clock64() - t0 > p.timeout_ticks) {
          set_status(p, 24u /* MER_ERR_RUNTIME_INVARIANT: dependency timeout */);
          __hip_atomic_store(p.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
      }
    }
  }
  ok = __shfl(ok, 0, 64);
  compiler_fence();
  return ok != 0;
}

// Publish this wave's device-scope stores, then count one arrival.
__device__ __forceinline__ void signal(uint32_t *ctr) {
  drain_stores();
  if (lane_id() == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  compiler_fence();
}

// Publish, count one arrival, and report whether this was the last of
// `expected` (whose stores are then all visible to device-scope loads).
__device__ __forceinline__ bool arrive_last(uint32_t *ctr, uint32_t expected) {
  drain_stores();
  uint32_t old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  compiler_fence();
  return old + 1 == expected;
}

// Count one arrival without draining this wave's stores first (for counts
// whose arrivals publish nothing the last arrival reads).
__device__ __forceinline__ bool arrive_last_nodrain(uint32_t *ctr, uint32_t expected) {
  uint32_t old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  compiler_fence();
  return old + 1 == expected;
}

// Release flag k of (layer, token): its own 256-byte line; holds the epoch
// of the last launch whose layer was complete for that token.
__device__ __forceinline__ uint64_t *release_flag(const DecodeParams &p, uint32_t layer, uint32_t t, uint32_t k) {
  return p.release + (((size_t)layer * p.n_tok + t) * kReleaseFan + k) * kFlagStride;
}

// Release flag k of the h slice (layer, instance, column slice), set when
// all of the slice's h tiles are packed.
__device__ __forceinline__ uint64_t *gd_flag(const DecodeParams &p, uint32_t layer, uint32_t inst, uint32_t ds,
                                             uint32_t k) {
  return p.gd_release + ((((size_t)layer * p.n_inst + inst) * p.d_slices + ds) * kReleaseFan + k) * kFlagStride;
}

// Optional per-item trace, 8 x u64 per item: {item << 32 | XCC << 16 | low
// HW_ID bits, start, inputs ready, digits fetched, walk done, arrived
// (D items), end, combined (combining D items)} in wall-clock ticks
// (records beyond trace_cap are dropped; unset marks are 0).
struct TraceMarks {
  uint64_t start, ready, fetched, walked, arrived, extra;
};
__device__ __forceinline__ uint64_t trace_now(const DecodeParams &p) { return p.trace ? wall_clock64() : 0; }
__device__ __forceinline__ void trace_item(const DecodeParams &p, uint64_t gi, const TraceMarks &m) {
  if (!p.trace || lane_id() != 0 || gi >= p.trace_cap) return;
  uint64_t *r = p.trace + gi * 8;
  uint32_t hw = 0, xcc = 0;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  r[0] = (gi << 32) | (hw & 0xffffu) | ((xcc & 0xfu) << 16);
  r[1] = m.start;
  r[2] = m.ready;
  r[3] = m.fetched;
  r[4] = m.walked;
  r[5] = m.arrived;
  r[6] = wall_clock64();
  r[7] = m.extra;
}

// One step of the transposed row reduction at lane distance D: lanes whose
// bit D is clear keep a, the others keep b, and each adds its partner's
// copy (lane l^D for D >= 8, the mirror lane 7-l of an 8-lane half for
// D = 4), so the result holds a partial sum of a on the lower lanes of each
// 2D block and of b on the upper ones, each spread over D lanes.  D = 32
// and 16 use the lane swaps across 32- and 16-lane halves, D <= 8 DPP.
template <int D>
__device__ __forceinline__ float split_sum(float a, float b) {
  if constexpr (D == 32 || D == 16) {
    const auto r = D == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false)
                           : __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    static_assert(D == 8 || D == 4, "split distance");
    constexpr int kCtrl = D == 8 ? 0x128 /* row_ror:8 */ : 0x141 /* row_half_mirror */;
    const bool hi = threadIdx.x & D;
    const float keep = hi ? b : a, send = hi ? a : b;
    return keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), kCtrl, 0xf, 0xf, true));
  }
}

// Sum over each aligned block of N lanes (N = 4, 8 or 16), on every lane of
// the block, by DPP adds.  Every pattern used reads a lane inside the same
// row, so bound_ctrl (zero for a source outside the row) never applies; it
// is set because it lets the compiler fold each move into its add.
template <int N>
__device__ __forceinline__ float span_sum(float v) {
  static_assert(N == 4 || N == 8 || N == 16, "span");
  auto add = [](float x, auto ctrl) {
    return x + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, true));
  };
  if constexpr (N == 16) {
    v = add(v, std::integral_constant<int, 0x128>{});  // row_ror:8
    v = add(v, std::integral_constant<int, 0x124>{});  // row_ror:4
  } else if constexpr (N == 8) {
    v = add(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  }
  v = add(v, std::integral_constant<int, 0x4e>{});  // quad_perm [2,3,0,1]
  v = add(v, std::integral_constant<int, 0xb1>{});  // quad_perm [1,0,3,2]
  return v;
}

// Quantise `nblocks` (<= 64 / groups) blocks of x into digit planes in line
// format (dword 24 = scale, dwords 25..26 = launch epoch); one wave, lane =
// group.  DEV: x is read with device-scope loads (it may have been written
// by another wave of this launch); otherwise x is in LDS.
template <int FMT, bool DEV, bool Q8ACT = false>
__device__ __forceinline__ void pack_blocks(const float *x, uint32_t nblocks, uint32_t *dig, uint64_t epoch) {
  using D = DigitTraits<FMT>;
  const uint32_t g = lane_id();
  const bool valid = g < nblocks * D::kGroups;
  const uint32_t b = g / D::kGroups, m = g % D::kGroups;
  float v[D::kGroupElems];
  float amax = 0.f;
  int finite = 1;
  if (valid) {
    const float *xb = x + (size_t)b * 32;
#pragma unroll
    for (int i = 0; i < D::kGroupElems; ++i) {
      const float *src = xb + group_elem<FMT>((int)m, i);
      v[i] = DEV ? ld_dev(src) : *src;
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
    const BlockScale bs = Q8ACT ? make_block_scale_q8(amax) : make_block_scale(amax, finite != 0);
    uint32_t plane[D::kPlanes];
    pack_group<FMT, Q8ACT>(v, bs.inv, plane);
    uint32_t *line = dig + (size_t)b * kLineDwords;
#pragma unroll
    for (int k = 0; k < D::kPlanes; ++k) st_dev(line + k * D::kGroups + m, plane[k]);
    if (m == 0) {  // scale and launch epoch, one 16-byte store
      const uint32_t tail[4] = {__float_as_uint(bs.s), (uint32_t)epoch, (uint32_t)(epoch >> 32), 0u};
      __hip_atomic_store(reinterpret_cast<uint64_t *>(line + kBlockDigitDwords),
                         (uint64_t)tail[0] | ((uint64_t)tail[1] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(reinterpret_cast<uint64_t *>(line + kBlockDigitDwords + 2),
                         (uint64_t)tail[2] | ((uint64_t)tail[3] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Streaming walk of one 32-row tile: lane groups of G lanes, R rows per
// pass, S weight streams (2 = gate and up).  Weight loads are raw buffer
// loads: a lane without a chunk gets an offset past the buffer's range and
// reads zeros, so the load sequence is branch-free and the compiler can
// keep exactly the next passes' loads outstanding.  The V = S*R sums of a
// pass are reduced transposed: split steps at lane distances G/2, G/4, ...
// halve the values per lane and the lanes per value together, so that
// after log2(V) steps each lane holds one value spread over G/V lanes, and
// DPP adds finish it (10 VALU ops for V = 4 on 64 or 32 lanes, against 44
// for four separate group sums).  `emit(writer, row, s, sum)` then runs on
// every lane with the lane's row and stream; one lane per value is the
// writer.
constexpr uint32_t kNoChunk = 0x80000000u;  // beyond num_records: loads return 0

template <int FMT, int G, int R, int S, int NB, bool Q8ACT>
struct TileWalk {
  using T = FmtTraits<FMT>;
  static constexpr int kGroups = 64 / G;
  static constexpr int kRows = R;  // rows of a lane group per pass
  static constexpr uint32_t kStep = R * kGroups;
  static constexpr uint32_t kPasses = kTileRows / kStep;
  static_assert(kTileRows % kStep == 0 && kPasses % NB == 0, "passes must tile 32 rows in whole buffer rounds");
  static constexpr int kV = S * R;       // sums per lane and pass
  static constexpr int kSpan = G / kV;   // lanes over which one reduced sum lies
  static_assert((kV & (kV - 1)) == 0 && kSpan >= 4 && kSpan <= 16, "reduction shape");
  using WBuf = uint32_t[S][R][T::kChunkDwords];

  __amdgpu_buffer_rsrc_t rsrc[S];
  uint32_t row_bytes;
  uint32_t voff;    // byte offset of the lane's chunk in row r_base (kNoChunk if none)
  uint32_t r_base;  // first row of this lane group's first pass
  uint32_t my_row;  // r_base + the row of the sum this lane ends with
  int my_s;         // stream of that sum
  bool writer;      // first lane of its sum's span

  __device__ __forceinline__ void init(const uint8_t *const (&base)[S], uint32_t row_bytes_, uint32_t chunk,
                                       bool valid, uint32_t r_base_) {
#pragma unroll
    for (int s = 0; s < S; ++s)
      rsrc[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base[s]), 0, 0x7fffffff, 0x00020000);
    row_bytes = row_bytes_;
    r_base = r_base_;
    voff = valid ? r_base_ * row_bytes_ + chunk * (uint32_t)T::kChunkBytes : kNoChunk;
    // value index k = s*R + j: the lane's bits at the split distances,
    // most significant first
    const uint32_t k = (threadIdx.x % G) / kSpan;
    my_row = r_base_ + k % R;
    my_s = (int)(k / R);
    writer = threadIdx.x % kSpan == 0;
  }

  __device__ __forceinline__ float reduce(float (&v)[kV]) const {
    if constexpr (kV >= 2) {
#pragma unroll
      for (int i = 0; i < kV / 2; ++i) v[i] = split_sum<G / 2>(v[i], v[i + kV / 2]);
    }
    if constexpr (kV >= 4) {
#pragma unroll
      for (int i = 0; i < kV / 4; ++i) v[i] = split_sum<G / 4>(v[i], v[i + kV / 4]);
    }
    if constexpr (kV >= 8) {
#pragma unroll
      for (int i = 0; i < kV / 8; ++i) v[i] = split_sum<G / 8>(v[i], v[i + kV / 8]);
    }
    static_assert(kV <= 8, "at most three split steps");
    return span_sum<kSpan>(v[0]);
  }

  __device__ __forceinline__ void load(uint32_t pass, WBuf &wb) const {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const uint32_t off = voff + (pass * kStep + j) * row_bytes;
        constexpr int kVec = T::kChunkDwords / 4;
#pragma unroll
        for (int v = 0; v < kVec; ++v) {
          const uint4 q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc[s], off + 16 * v, 0, 0));
          wb[s][j][4 * v] = q.x;
          wb[s][j][4 * v + 1] = q.y;
          wb[s][j][4 * v + 2] = q.z;
          wb[s][j][4 * v + 3] = q.w;
        }
        wb[s][j][4 * kVec] = __builtin_amdgcn_raw_buffer_load_b32(rsrc[s], off + 16 * kVec, 0, 0);
      }
  }

  template <class Emit>
  __device__ __forceinline__ void compute(uint32_t pass, WBuf &wb, const uint32_t *xd, const float *xsc,
                                          Emit &&emit) const {
    float v[kV];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < R; ++j) v[s * R + j] = chunk_idot<FMT, Q8ACT>(wb[s][j], xd, xsc);
    emit(writer, my_row + pass * kStep, my_s, reduce(v));
  }

  // Issue the loads of passes 0 .. NB-1 into the NB buffers.
  __device__ __forceinline__ void prefetch(WBuf (&w)[NB]) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) load(b, w[b]);
  }

  // Passes 0 .. NB-1 must already be loaded (prefetch).  Each buffer is
  // refilled with the pass NB ahead as soon as it has been consumed, so NB-1
  // passes stay in flight while one is computed.  The scheduling barriers
  // keep the compiler from hoisting one buffer's dot products above another
  // buffer's loads, which would make each pass wait for loads issued just
  // before it.
  template <class Emit>
  __device__ __forceinline__ void run(WBuf (&w)[NB], const uint32_t *xd, const float *xsc, Emit &&emit) const {
#pragma unroll 1
    for (uint32_t pass = 0; pass + NB < kPasses; pass += NB) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        compute(pass + b, w[b], xd, xsc, emit);
        __builtin_amdgcn_sched_barrier(0);
        load(pass + NB + b, w[b]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) compute(kPasses - NB + b, w[b], xd, xsc, emit);
  }
};

// Fetch the 48 digit dwords and 2 scales of chunk `c` (blocks block0 and
// block0 + 1) of a packed vector in line format.  The lines were written in
// this launch by waves that published a counter this wave has waited on,
// and were not read in this launch before that.  Ordinary cached loads let
// each XCD's L2 serve the many waves that read the same vector instead of
// sending every read to the one memory channel that holds it.  A cache may
// still hold a copy of a line from an earlier launch (another XCD's
// device-scope stores do not touch this XCD's L2): such a copy carries an
// older epoch, and the lane then reads the line again with device-scope
// loads, which bypass the non-coherent caches.
__device__ __forceinline__ void fetch_digits(const uint32_t *dig, size_t block0, bool valid, uint64_t epoch,
                                             uint32_t (&xd)[2 * kBlockDigitDwords], float (&xsc)[2]) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(dig), 0, 0x7fffffff, 0x00020000);
  const uint32_t voff = valid ? (uint32_t)(block0 * kLineDwords * 4u) : kNoChunk;
  uint32_t tag_lo[2], tag_hi[2];
  auto fetch = [&](auto aux) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int k = 0; k < kBlockDigitDwords / 4; ++k) {
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 4u * (b * kLineDwords + 4 * k), 0, decltype(aux)::value));
        xd[b * kBlockDigitDwords + 4 * k] = v.x;
        xd[b * kBlockDigitDwords + 4 * k + 1] = v.y;
        xd[b * kBlockDigitDwords + 4 * k + 2] = v.z;
        xd[b * kBlockDigitDwords + 4 * k + 3] = v.w;
      }
      const uint4 st = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 4u * (b * kLineDwords + kBlockDigitDwords), 0,
                                                       decltype(aux)::value));
      xsc[b] = __uint_as_float(st.x);
      tag_lo[b] = st.y;
      tag_hi[b] = st.z;
    }
  };
  fetch(std::integral_constant<int, 0>{});
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt unchanged
  const uint32_t e_lo = (uint32_t)epoch, e_hi = (uint32_t)(epoch >> 32);
  const bool stale = valid && ((tag_lo[0] ^ e_lo) | (tag_hi[0] ^ e_hi) | (tag_lo[1] ^ e_lo) | (tag_hi[1] ^ e_hi)) != 0u;
  if (__builtin_amdgcn_ballot_w64(stale)) {
    if (stale) fetch(std::integral_constant<int, 16 /* SC1: device scope */>{});
    // Waiting here, once, also keeps the compiler's wait-count analysis from
    // treating the digits as outstanding at the loop header of the walk
    // (which would drain every weight load on each iteration).
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
}

}  // namespace

// PAIR: workgroups of two waves taking items 2u and 2u+1 of unit u.  Used
// when gate/up rows are cut into two column slices (narrow layers, single
// experts): the slices of a tile are consecutive items, so they meet in one
// workgroup and their partial sums are added in LDS instead of going
// through memory and an arrival count (one round trip instead of three).
template <int FMT, int GG, int GD, bool PAIR, bool Q8ACT>
__global__ __launch_bounds__(PAIR ? 128 : 64) __attribute__((amdgpu_waves_per_eu(FMT == FMT_Q4_0 ? 3 : 2))) void decode_kernel(DecodeParams p) {
  constexpr uint32_t kW = PAIR ? 2 : 1;  // waves per workgroup
  const uint32_t wv = PAIR ? (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / 64) : 0u;
  __shared__ float s_h_all[kW][kTileRows];
  __shared__ float s_gu_all[kW][2 * kTileRows];  // gate and up row sums of a single-slice G item
  __shared__ float s_pair[PAIR ? 2 : 1][2 * kTileRows];  // a paired G tile's slice sums
  float *s_h = s_h_all[wv];
  float *s_gu = s_gu_all[wv];
  const uint32_t lane = lane_id();
  using D = DigitTraits<FMT>;
  constexpr uint32_t kPackBlocks = 64 / D::kGroups;
  // Weight passes kept in registers per wave.  Two keep the kernel at 166
  // VGPRs, three waves per SIMD: a third resident wave per SIMD (the next
  // layer's items prefetching, a second G or D wave) hides more latency than
  // two more passes in flight per wave would.
  constexpr int kBuffers = 2;

  // Every wave reads the launch's epoch; the word changes only after the
  // last wave has left (below).
  const uint64_t epoch_v = ld_dev(p.epoch_word);
  const uint64_t epoch = join_u32((uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(epoch_v >> 32)),
                                  (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)epoch_v));
  // Item i goes to workgroup i mod grid.  An item waits only on items with
  // smaller indices.  The walk drains as long as no wave waits forever on an
  // item of a workgroup that never becomes resident: the host orders all
  // decode launches of a device one after another (launch_planned), so no
  // other persistent grid of this library overlaps this one, and workgroups
  // still pending behind other kernels become resident as those finish.
  const uint64_t n_units = (p.total_items + kW - 1) / kW;
  for (uint32_t u = blockIdx.x; u < n_units; u += gridDim.x) {
    const uint32_t gi = u * kW + wv;
    if (gi >= p.total_items) continue;  // the other wave of a last, odd unit
    TraceMarks tm{};
    tm.start = trace_now(p);
    const uint32_t l = (uint32_t)(gi / p.items_per_layer);
    const uint32_t j = (uint32_t)(gi % p.items_per_layer);
    const LayerArgs &la = p.layers[l];
    uint32_t *cnt = p.counters + (size_t)l * p.cnt_per_layer;
    uint32_t *xq_dig = p.xq_dig + (size_t)l * p.n_tok * p.xblocks * kLineDwords;
    uint32_t *hq_dig = p.hq_dig + (size_t)l * p.n_inst * p.hblocks * kLineDwords;
    // layer input of token t
    const float *xsrc = (p.flags & kFlagChain) && l > 0 ? p.layers[l - 1].out : la.x;
    // Layer l-1's output for token t is complete: the last of its combines
    // has set the layer's release flags to this launch's epoch.  A waiter
    // polls one of kReleaseFan flags (by item), so hundreds of waiting waves
    // do not all poll the line the combines count on.
    auto wait_prev_layer = [&](uint32_t t) {
      if (l > 0) wait_flag(p, release_flag(p, l - 1, t, (uint32_t)(gi % kReleaseFan)), epoch, kNapFlag);
    };
    const bool route_after_prev = (p.flags & kFlagRouteAfterPrev) != 0;
    // Layer l's input digits of token t are complete.  Layer 0's are packed
    // by its P items; with combine packing, layer l > 0's input block b is
    // packed by the combine of tile b of layer l-1, so all of them are there
    // once every tile of layer l-1 is combined.
    auto wait_input = [&](uint32_t t) {
      if (l > 0 && p.combine_packs) wait_prev_layer(t);
      else wait_for(p, cnt + p.c_p + (size_t)t * kPollStride, p.p_items, kNapCounter);
    };
    // Under ROUTE_AFTER_PREV, G and D items touch their experts only once the
    // layer's input is packed (which implies layer l-1 is complete), so the
    // input packing does not queue behind every wave's weight prefetch.
    auto wait_input_packed = [&](uint32_t t) {
      if (l > 0) wait_input(t);
    };

    if (j < p.off_p) {
      // ---- R: report residency misses of the token's expert slots ---------
      // (G and D items resolve their blob themselves and treat a miss as a
      // zero expert, so nothing waits on this item.)
      const uint32_t t = j;
      if (route_after_prev) wait_prev_layer(t);
      // A zero-weight slot is skipped by the combine (engine.rs:5575-5580),
      // so its id is not checked (the router marks unused slots id -1, w 0).
      if (lane < p.top_k && !p.single) {
        const int32_t id = la.ids[t * p.top_k + lane];
        const bool unused = la.weights && la.weights[t * p.top_k + lane] == 0.0f;
        if (!unused && (id < 0 || (uint32_t)id >= la.table_len || !la.table[id]))
          set_status(p, 16u /* MER_ERR_RESIDENCY_MISS */);
      }
    } else if (j < p.off_g) {
      // ---- P: pack part of the token's layer input ------------------------
      const uint32_t idx = j - p.off_p;
      const uint32_t t = idx / p.p_items;
      const uint32_t part = idx % p.p_items;
      if (t < p.n_tok && (l == 0 || !p.combine_packs)) {  // else packed by layer l-1's combines (or padding)
        wait_prev_layer(t);  // layers run in order: layer l reads after layer l-1 wrote
        tm.ready = trace_now(p);
        const uint32_t b0 = part * kPackBlocks;
        const uint32_t nb = min(kPackBlocks, p.xblocks - b0);
        const size_t tb = (size_t)t * p.xblocks + b0;
        pack_blocks<FMT, true, Q8ACT>(xsrc + (size_t)t * p.d_model + (size_t)b0 * 32, nb, xq_dig + tb * kLineDwords, epoch);
        signal(cnt + p.c_p + (size_t)t * kPollStride);
      }
    } else if (j < p.off_d) {
      // ---- G: gate/up of one (slot, column slice, tile) -------------------
      const uint32_t idx = j - p.off_g;
      const uint32_t per_inst = p.g_tiles * p.g_slices;
      const uint32_t inst = idx / per_inst;
      const uint32_t tile = (idx % per_inst) / p.g_slices;
      const uint32_t gs = idx % p.g_slices;
      const uint32_t t = inst / p.top_k;
      if (route_after_prev) wait_input_packed(t);
      const uint8_t *expert = resolve_expert(p, la, inst);
      const uint32_t dslice = tile * 32 / (p.d_cps * 64);
      using W = TileWalk<FMT, GG, 2, 2, kBuffers, Q8ACT>;
      const uint32_t grp = lane / GG, gl = lane % GG;
      const uint32_t c_begin = gs * p.g_cps;
      const uint32_t c = c_begin + gl;
      const bool valid = expert && gl < p.g_cps && c < p.g_chunks;
      const uint8_t *const bases[2] = {expert, expert + p.proj_bytes};
      W walk;
      walk.init(bases, p.g_chunks * (uint32_t)FmtTraits<FMT>::kChunkBytes, c, valid, tile * kTileRows + grp * W::kRows);
      typename W::WBuf wbuf[kBuffers];
      walk.prefetch(wbuf);
      wait_input(t);
      tm.ready = trace_now(p);
      uint32_t xd[2 * kBlockDigitDwords];
      float xsc[2];
      prio_hi();
      fetch_digits(xq_dig, (size_t)t * p.xblocks + 2 * (size_t)c, valid, epoch, xd, xsc);
      prio_lo();
      tm.fetched = trace_now(p);
      float *gpart = p.gpart + (((size_t)l * p.n_inst + inst) * p.g_slices + gs) * 2 * p.d_ff;
      const bool single_slice = p.g_slices == 1;
      auto emit = [&](bool writer, uint32_t r, int s, float a) {
        if (writer) {
          if (single_slice) s_gu[s * kTileRows + r - tile * kTileRows] = a;
          else if (PAIR) s_pair[wv][s * kTileRows + r - tile * kTileRows] = a;
          else st_dev(gpart + (size_t)s * p.d_ff + r, a);
        }
      };
      walk.run(wbuf, xd, xsc, emit);
      prio_hi();
      tm.walked = trace_now(p);
      bool pack = single_slice;
      if (single_slice) {
        wave_lds_sync();
        if (lane < kTileRows) s_h[lane] = expert ? silu_mul(s_gu[lane], s_gu[kTileRows + lane], p.swiglu_limit) : 0.f;
      } else if (PAIR) {
        // both waves of the workgroup hold the two slices of this tile
        __syncthreads();
        pack = wv == 0;
        if (pack && lane < kTileRows)
          s_h[lane] = expert ? silu_mul(s_pair[0][lane] + s_pair[1][lane],
                                        s_pair[0][kTileRows + lane] + s_pair[1][kTileRows + lane], p.swiglu_limit)
                             : 0.f;
        __syncthreads();  // s_pair is free for the next unit
      } else {
        pack = arrive_last(cnt + p.c_ga + (size_t)inst * p.g_tiles + tile, p.g_slices);
        if (pack && lane < kTileRows) {
          const size_t base = ((size_t)l * p.n_inst + inst) * p.g_slices * 2 * p.d_ff;
          const uint32_t r = tile * kTileRows + lane;
          float g = 0.f, u = 0.f;
          for (uint32_t s = 0; s < p.g_slices; ++s) {
            g += ld_dev(p.gpart + base + (size_t)s * 2 * p.d_ff + r);
            u += ld_dev(p.gpart + base + (size_t)s * 2 * p.d_ff + p.d_ff + r);
          }
          s_h[lane] = silu_mul(g, u, p.swiglu_limit);
        }
      }
      if (pack) {
        wave_lds_sync();
        const size_t hb = (size_t)inst * p.hblocks + tile;
        pack_blocks<FMT, false, Q8ACT>(s_h, 1, hq_dig + hb * kLineDwords, epoch);
        uint32_t *gd = cnt + p.c_gd + ((size_t)inst * p.d_slices + dslice) * kPollStride;
        if (p.gd_release) {
          // the last h tile of the slice releases its D items
          const uint32_t tiles = min(p.d_cps * 2, p.g_tiles - dslice * p.d_cps * 2);
          if (arrive_last(gd, tiles) && lane < kReleaseFan) st_dev(gd_flag(p, l, inst, dslice, lane), epoch);
        } else {
          signal(gd);
        }
      }
    } else {
      // ---- D: down of one (slot, column slice, tile) + combine -------------
      const uint32_t idx = j - p.off_d;
      if (idx >= p.n_inst * p.d_slices * p.d_tiles) continue;  // padding item
      const uint32_t per_tok = p.d_tiles * p.top_k * p.d_slices;
      const uint32_t t = idx / per_tok;
      const uint32_t rem = idx % per_tok;
      const uint32_t tile = rem / (p.top_k * p.d_slices);
      const uint32_t slot = (rem / p.d_slices) % p.top_k;
      const uint32_t ds = rem % p.d_slices;
      const uint32_t inst = t * p.top_k + slot;
      if (route_after_prev) wait_input_packed(t);
      const uint8_t *expert = resolve_expert(p, la, inst);
      using W = TileWalk<FMT, GD, (GD == 16 ? 2 : 4), 1, kBuffers, Q8ACT>;
      const uint32_t grp = lane / GD, gl = lane % GD;
      const uint32_t c = ds * p.d_cps + gl;
      const bool valid = expert && gl < p.d_cps && c < p.d_chunks;
      const uint8_t *const bases[1] = {expert + 2 * p.proj_bytes};
      W walk;
      walk.init(bases, p.d_chunks * (uint32_t)FmtTraits<FMT>::kChunkBytes, c, valid,
                tile * kTileRows + grp * W::kRows);
      typename W::WBuf wbuf[kBuffers];
      walk.prefetch(wbuf);
      // the h planes of this column slice
      const uint32_t first_tile = ds * p.d_cps * 2;
      const uint32_t n_tiles = min(p.d_cps * 2, p.g_tiles - first_tile);
      if (p.gd_release) wait_flag(p, gd_flag(p, l, inst, ds, (uint32_t)(gi % kReleaseFan)), epoch, kNapFlag);
      else wait_for(p, cnt + p.c_gd + ((size_t)inst * p.d_slices + ds) * kPollStride, n_tiles, kNapCounter);
      tm.ready = trace_now(p);
      uint32_t xd[2 * kBlockDigitDwords];
      float xsc[2];
      prio_hi();
      fetch_digits(hq_dig, (size_t)inst * p.hblocks + 2 * (size_t)c, valid, epoch, xd, xsc);
      prio_lo();
      tm.fetched = trace_now(p);
      float *part = p.partial + (((size_t)l * p.n_inst + inst) * p.d_slices + ds) * p.d_model;
      // Row sums go to LDS, then out as one 128-byte store.  The slot weight
      // is applied here; a zero-weight slot contributes exactly nothing, as
      // the engine skips it (engine.rs:5575-5580).
      const float w_slot = la.weights ? la.weights[t * p.top_k + slot] : 1.0f;
      auto emit = [&](bool writer, uint32_t r, int, float a) {
        if (writer) s_h[r - tile * kTileRows] = a;
      };
      walk.run(wbuf, xd, xsc, emit);
      prio_hi();
      tm.walked = trace_now(p);
      wave_lds_sync();
      // What a combine of this tile adds to the sum is already final: the
      // residual or accumulated output (written by layer l-1, complete before
      // any item of this layer ran) and the caller's next-layer input.  Every
      // D item loads it now, so the drain of its arrival covers the latency
      // and the combine waits on one round trip only.
      const bool pack_next = p.combine_packs && l + 1 < p.n_layers;
      float base = 0.f, next_x = 0.f;
      if (lane < kTileRows) {
        const uint32_t r = tile * kTileRows + lane;
        if (p.flags & kFlagResidual) base = ld_dev(xsrc + (size_t)t * p.d_model + r);
        else if (p.flags & kFlagAccumulate) base = ld_dev(la.out + (size_t)t * p.d_model + r);
        if (pack_next && !(p.flags & kFlagChain)) next_x = p.layers[l + 1].x[(size_t)t * p.d_model + r];
        const float y = s_h[lane];
        st_dev(part + tile * kTileRows + lane, (la.weights && w_slot == 0.0f) ? 0.0f : w_slot * y);
      }
      const bool last = arrive_last(cnt + p.c_da + (size_t)t * p.d_tiles + tile, p.top_k * p.d_slices);
      tm.arrived = trace_now(p);
      if (last) {
        // out = [x +] sum over slots i (and column slices) of w_i * y_i, in
        // slot order (combine_outputs_into, inference.rs:4472-4491).  All
        // device-scope loads are issued before any is used, so the combine
        // costs one round trip.
        if (lane < kTileRows) {
          const uint32_t r = tile * kTileRows + lane;
          float *o = la.out + (size_t)t * p.d_model + r;
          const uint32_t n_parts = p.top_k * p.d_slices;
          const float *pp = p.partial + ((size_t)l * p.n_inst + (size_t)t * p.top_k) * p.d_slices * p.d_model + r;
          float acc = 0.f;
          if (n_parts <= kCombineBatch) {
            float v[kCombineBatch];
#pragma unroll
            for (uint32_t k = 0; k < kCombineBatch; ++k) v[k] = k < n_parts ? ld_dev(pp + (size_t)k * p.d_model) : 0.f;
#pragma unroll
            for (uint32_t k = 0; k < kCombineBatch; ++k)
              if (k < n_parts) acc += v[k];
          } else {
            for (uint32_t k = 0; k < n_parts; ++k) acc += ld_dev(pp + (size_t)k * p.d_model);
          }
          const float val = (p.flags & (kFlagResidual | kFlagAccumulate)) ? base + acc : acc;
          st_dev(o, val);
          if (pack_next) s_h[lane] = (p.flags & kFlagChain) ? val : next_x;
        }
        if (pack_next) {
          // block `tile` of layer l+1's input, the tile just combined (chained)
          // or the caller's next input, into layer l+1's digit lines
          wave_lds_sync();
          uint32_t *next_dig = p.xq_dig + ((size_t)(l + 1) * p.n_tok * p.xblocks + (size_t)t * p.xblocks + tile) * kLineDwords;
          pack_blocks<FMT, false, Q8ACT>(s_h, 1, next_dig, epoch);
        }
        tm.extra = trace_now(p);
        // the last layer's release flags have no reader
        if (l + 1 < p.n_layers && arrive_last(cnt + p.c_c + (size_t)t * kPollStride, p.d_tiles) &&
            lane < kReleaseFan)
          st_dev(release_flag(p, l, t, lane), epoch);
        compiler_fence();
      }
    }
    trace_item(p, gi, tm);
    prio_lo();
  }

  // The last wave out (every wave has read the epoch) zeroes the counters
  // and gives the next launch on
  // this workspace a fresh epoch, unique on the device: the top bit set
  // keeps it apart from the host-chosen first epochs of workspaces.
  const uint32_t n_waves = gridDim.x * kW;
  const uint32_t grp = (blockIdx.x * kW + wv) % kExitGroups;
  const uint32_t in_grp = n_waves / kExitGroups + (grp < n_waves % kExitGroups ? 1u : 0u);
  uint32_t *grp_ctr = p.exit_groups + (size_t)grp * kPollStride;
  // The group arrival drains: this wave's last counter atomics (issued
  // without waiting for a return) land before the last wave zeroes the
  // counters.  What the last waves store after that (the group counter's
  // reset, the zeroed counters, the next epoch) needs no drain: the next
  // launch on this workspace starts after this kernel has completed.
  if (!arrive_last(grp_ctr, in_grp)) return;
  if (lane == 0) st_dev(grp_ctr, 0u);
  if (arrive_last_nodrain(p.exit_count, min(n_waves, kExitGroups))) {
    for (uint32_t i = lane; i < p.n_counters; i += 64) st_dev(p.counters + i, 0u);
    if (lane == 0) {
      st_dev(p.abort_flag, 0u);
      const uint64_t seq = __hip_atomic_fetch_add(&g_epoch_seq, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      st_dev(p.epoch_word, (uint64_t)((1ull << 63) | (seq + 1)));
      st_dev(p.exit_count, 0u);
    }
  }
}

// Prepares decode scratch whose earlier contents belong to calls of other
// shapes (the no-alloc entry point's static array): zeroes n_ctl words at
// ctl (exit count, abort flag, exit-group counters) and n_zero words at zero (counters, release
// flags), and gives an epoch word that has never been used (0) its first
// epoch.
__global__ __launch_bounds__(256) void decode_scratch_prep_kernel(uint32_t *ctl, uint32_t n_ctl, uint32_t *zero,
                                                                  size_t n_zero, uint64_t *epoch_word) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n_ctl) ctl[i] = 0u;
  if (i < n_zero) zero[i] = 0u;
  if (i == 0 && *epoch_word == 0) {
    const uint64_t seq = __hip_atomic_fetch_add(&g_epoch_seq, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *epoch_word = (uint64_t)((1ull << 63) | (seq + 1));
  }
}

hipError_t launch_decode_scratch_prep(uint32_t *ctl, uint32_t n_ctl, uint32_t *zero, size_t n_zero,
                                      uint64_t *epoch_word, hipStream_t st) {
  const size_t n = n_zero > n_ctl ? n_zero : n_ctl;
  hipLaunchKernelGGL(decode_scratch_prep_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, ctl, n_ctl,
                     zero, n_zero, epoch_word);
  return hipGetLastError();
}

template <int FMT, int GG, int GD, bool PAIR, bool Q8ACT>
static const void *decode_fn() {
  return reinterpret_cast<const void *>(&decode_kernel<FMT, GG, GD, PAIR, Q8ACT>);
}

template <int FMT, int GG, bool PAIR, bool Q8ACT>
static const void *decode_fn_gd(int gd) {
  if (gd == 16) return decode_fn<FMT, GG, 16, PAIR, Q8ACT>();
  if (gd == 32) return decode_fn<FMT, GG, 32, PAIR, Q8ACT>();
  return decode_fn<FMT, GG, 64, PAIR, Q8ACT>();
}

// Paired workgroups serve gate/up rows cut into two slices of at most 32
// chunks (GG 16 or 32); single-wave workgroups serve everything else.
template <int FMT, bool Q8ACT>
static const void *decode_fn_fmt(int gg, int gd, bool pair) {
  if (pair) return gg == 16 ? decode_fn_gd<FMT, 16, true, Q8ACT>(gd) : decode_fn_gd<FMT, 32, true, Q8ACT>(gd);
  if (gg == 16) return decode_fn_gd<FMT, 16, false, Q8ACT>(gd);
  if (gg == 32) return decode_fn_gd<FMT, 32, false, Q8ACT>(gd);
  return decode_fn_gd<FMT, 64, false, Q8ACT>(gd);
}

// q8act: Candle's Q8_0 activations (QMatMul), Q4_0 weights only.
const void *decode_kernel_fn(int fmt, int gg, int gd, bool pair, bool q8act) {
  if (fmt != FMT_Q4_0) return decode_fn_fmt<FMT_Q8_0, false>(gg, gd, pair);
  return q8act ? decode_fn_fmt<FMT_Q4_0, true>(gg, gd, pair) : decode_fn_fmt<FMT_Q4_0, false>(gg, gd, pair);
}

hipError_t launch_decode(const void *fn, uint32_t grid, uint32_t waves_per_group, const DecodeParams &p,
                         hipStream_t st) {
  void *args[] = {const_cast<DecodeParams *>(&p)};
  return hipLaunchKernel(fn, dim3(grid), dim3(64 * waves_per_group), args, 0, st);
}

}  // namespace mer
