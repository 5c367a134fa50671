// mer_grouped.hip -- grouped per-expert path for multi-token batches (gfx950).
//
// A prefill-sized batch routes many tokens to the same expert, so each
// expert's weights can be read once for all of its tokens.  That turns
// the per-expert work into a real dense contraction: [rows x K] weights by
// [K x tokens], run on int8 MFMA (v_mfma_i32_16x16x32_i8, K = 32 = one
// GGUF block).  Reference semantics are those of the decode path: every
// routed (token, slot) pair computes y = W_down (silu(W_gate x) * (W_up x))
// (inference.rs:3291-3306 / :3636-3746) and the token's output is
// [x +] sum_i w_i y_i in slot order (combine_outputs_into,
// inference.rs:4472-4491; the WeightedInto loop, engine.rs:5548-5639).
//
// Launches, all on the caller's stream:
//   group_kernel   block 0 groups the routed pairs by expert (counting
//                  sort) and emits token tiles of <= 16 pairs per expert;
//                  the other blocks quantise x into 24-bit digit records
//                  (three base-256 planes, below)
//   proj_kernel<FUSED>  one workgroup per (token tile, 32 rows of d_ff):
//                  gate and up rows for the tile's tokens, SiLU * up, h
//                  quantised per 32-element block
//   proj_kernel<!FUSED> one workgroup per (token tile, 64 rows of d_model):
//                  down rows -> w_i * y_i per pair
//   combine_kernel out[t] = [x +] sum over slots in slot order
//
// Numerics.  The weights are int8 (Q8_0 q, or Q4_0 q-8) with one f16
// scale per 32-weight block.  Each 32-element block b of an input vector
// (x, or h for the down projection) is held as s_b * v with
// s_b = max|x_b| / 8355711 and v = round(x / s_b), split into three signed
// base-256 digits v = v0 + 256 v1 + 65536 v2 (the bytes of v + 0x808080
// with their top bits flipped).  Per block, MFMA gives the exact int32
// sums Pk = sum q*vk (|Pk| < 2^19); P1 + 256 P2 is exact in int32, and the
// block contributes (256 (P1 + 256 P2) + P0) * d_w * s_b, formed in f32,
// to an f32 accumulator.  The representation error of v is at most 2^-24
// of the block's largest |x| (an f32 rounding of that element); non-finite
// inputs give a NaN scale, so NaN propagates.
//
// Operand layout of v_mfma_i32_16x16x32_i8: lane l holds 8 int8 of A row
// (l % 16) and of B column (l % 16), covering the same 8 of the block's 32
// k-indices (chosen by l / 16) in A and B; output lane l holds rows
// 4 (l / 16) + i, i = 0..3, of column l % 16.  Weights are staged through
// LDS as [row][block][32 int8] (rows padded to spread banks) plus f32
// scales [block][row]; the input digits are stored per (vector, block) as
// 4 groups x {8 bytes v0, 8 bytes v1, 8 bytes v2, f32 scale, pad}, so a
// lane reads the B operands of its k-group and the block scale from one
// 32-byte record.
#include "mer_internal.hpp"

namespace mer {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kGTok = 16;           // pairs per token tile (MFMA N)
constexpr int kGWavesPerEu = 4;
// Workgroup geometry: four waves, RT row tiles of 16 rows (RT = 4 or 8),
// stages of 32 / RT blocks, so every stage holds the same 256 two-block
// chunks (one per thread) whatever RT is.  Each wave computes every row
// tile for its 32 / (4 RT) blocks of the stage: with RT = 8 a B operand
// (one pair column's digit records of one block) serves twice as many
// weight rows, which halves the B bytes loaded per weight byte.
template <int RT>
struct GGeom {
  static constexpr uint32_t kRows = 16 * RT;                       // weight rows per workgroup
  static constexpr uint32_t kStageBlocks = 32 / RT;                // K blocks per stage
  static constexpr uint32_t kStageChunks = kStageBlocks / 2;       // two-block chunks per row per stage
  static constexpr int kWaveBlocks = (int)(kStageBlocks / 4);      // blocks of a stage per wave
  static constexpr uint32_t kRowStride = kStageBlocks * 32 + 16;   // LDS bytes per staged row (padded)
  // scales [block][row]; RT = 4 pads the row to spread the stores' banks,
  // RT = 8 keeps two slabs within a quarter of the CU's LDS
  static constexpr uint32_t kScaleStride = RT == 4 ? kRows + 4 : kRows;
  static_assert(kRows * kStageChunks == 256, "one chunk per thread and stage");
  static_assert(kWaveBlocks >= 1, "every wave has a block in every stage");
};
constexpr float kGIntMax = 8355711.0f;   // |v| bound (0x7f7f7f): v + 0x808080 stays in 24 bits
constexpr uint32_t kGRec = 8;            // dwords per (vector, block, k-group) record: 3 digit planes, scale, pad
constexpr uint32_t kNoChunkG = 0x80000000u;

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

__device__ __forceinline__ void record_status(uint32_t *status, uint32_t code) { atomicCAS(status, 0u, code); }

__device__ __forceinline__ bool pair_valid(const GroupedParams &p, uint32_t pair, const uint8_t **blob) {
  if (p.weights && p.weights[pair] == 0.0f) return false;  // skipped by the combine (engine.rs:5575-5580)
  const int32_t id = p.ids[pair];
  if (id < 0 || (uint32_t)id >= p.table_len) return false;
  const uint8_t *b = reinterpret_cast<const uint8_t *>(p.table[id]);
  if (blob) *blob = b;
  return b != nullptr;
}

// Quantise 8 elements (one MFMA k-group) of a block whose 4 groups sit in
// 4 adjacent lanes (lane & 3 = group): block max by shuffles, then one
// 32-byte record {v0[8], v1[8], v2[8], f32 block scale, 0}, so a reader
// gets a k-group's three digit planes and the block's scale with two
// 16-byte loads.  Only lanes with `store` write.
// q8: Candle's Q8_0 activation instead (QMatMul, MER_MOE_QMM): scale
// d = amax / 127 kept as f16, q = round(v / d) half away from zero (NaN ->
// 0), so |q| <= 128 lands in plane 0 and planes 1-2 are zero.
__device__ __forceinline__ void quant_group(const float (&v)[8], uint32_t *dst, bool store, bool q8) {
  float amax = 0.f;
  int finite = 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
    finite &= __builtin_isfinite(v[i]) ? 1 : 0;
  }
#pragma unroll
  for (int off = 1; off < 4; off <<= 1) {
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, off, 64));
    finite &= __shfl_xor(finite, off, 64);
  }
  float s, inv;
  if (q8) {
    const float d = amax / 127.0f;
    inv = d != 0.0f ? 1.0f / d : 0.0f;
    s = (float)(_Float16)d;
  } else if (!finite) {
    s = __builtin_nanf("");
    inv = 0.f;
  } else if (amax == 0.f) {
    s = 0.f;
    inv = 0.f;
  } else {
    s = amax / kGIntMax;
    inv = kGIntMax / amax;
  }
  uint32_t d[6] = {0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float q;
    if (q8) {
      q = __builtin_roundf(v[i] * inv);
      q = __builtin_isnan(q) ? 0.f : __builtin_fminf(__builtin_fmaxf(q, -128.0f), 127.0f);
    } else {
      q = __builtin_rintf(v[i] * inv);
      q = __builtin_fminf(__builtin_fmaxf(q, -kGIntMax), kGIntMax);
    }
    const uint32_t u = ((uint32_t)((int32_t)q + 0x808080)) ^ 0x808080u;  // three balanced digits
#pragma unroll
    for (int k = 0; k < 3; ++k) d[2 * k + (i >> 2)] |= ((u >> (8 * k)) & 0xffu) << (8 * (i & 3));
  }
  if (!store) return;
  uint4 *o = reinterpret_cast<uint4 *>(dst);
  o[0] = make_uint4(d[0], d[1], d[2], d[3]);
  o[1] = make_uint4(d[4], d[5], __float_as_uint(s), 0u);
}

// Block 0: group the routed pairs by expert.  Other blocks: quantise x.
__global__ __launch_bounds__(1024) void group_kernel(GroupedParams p) {
  if (blockIdx.x > 0) {
    const uint32_t g = (blockIdx.x - 1) * blockDim.x + threadIdx.x;  // (token, block, group)
    const uint32_t total = p.n_tok * p.xblocks * 4;
    // whole quads stay together for the shuffles; quads past the end idle
    const bool valid = g < total;
    const uint32_t tb = g / 4, m = g % 4;
    float v[8];
    if (valid) {
      const float4 a = *reinterpret_cast<const float4 *>(p.x + (size_t)tb * 32 + 8 * m);
      const float4 b = *reinterpret_cast<const float4 *>(p.x + (size_t)tb * 32 + 8 * m + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.f;
    }
    quant_group(v, p.xg + ((size_t)tb * 4 + m) * kGRec, valid, p.q8act != 0);
    return;
  }

  extern __shared__ uint32_t sh[];
  uint32_t *cnt = sh;                   // [table_len] pairs per expert, then offsets
  uint32_t *tcnt = sh + p.table_len;    // [table_len] tiles per expert, then offsets
  // [n_pairs] the pair's expert << 16 | its rank within the expert (both
  // < 4096), so the final scatter needs no second read of the routing
  uint32_t *pos = tcnt + p.table_len;
  __shared__ uint32_t part[1024 * 2];
  const uint32_t tid = threadIdx.x, nth = blockDim.x;
  for (uint32_t e = tid; e < p.table_len; e += nth) cnt[e] = 0u;
  __syncthreads();
  for (uint32_t q = tid; q < p.n_pairs; q += nth) {
    const uint8_t *blob = nullptr;
    const bool ok = pair_valid(p, q, &blob);
    p.pair_ok[q] = ok ? 1u : 0u;
    if (ok) {
      const uint32_t e = (uint32_t)p.ids[q];
      pos[q] = (e << 16) | atomicAdd(&cnt[e], 1u);
    } else {
      pos[q] = 0xffffffffu;
      if (!(p.weights && p.weights[q] == 0.0f)) record_status(p.status, 16u /* MER_ERR_RESIDENCY_MISS */);
    }
  }
  __syncthreads();
  // exclusive scans of pairs and tiles per expert: each thread owns a run
  // of consecutive experts
  const uint32_t per = (p.table_len + nth - 1) / nth;
  const uint32_t e0 = tid * per, e1 = min(p.table_len, e0 + per);
  uint32_t sp = 0, st = 0;
  for (uint32_t e = e0; e < e1; ++e) {
    const uint32_t c = cnt[e];
    sp += c;
    st += (c + kGTok - 1) / kGTok;
  }
  // Inclusive scan of (sp, st) over the block: within each wave by lane
  // shuffles, then over the wave totals (two barriers in all).
  uint32_t ip = sp, it = st;
  for (uint32_t off = 1; off < 64; off <<= 1) {
    const uint32_t a = __shfl_up(ip, off, 64), b = __shfl_up(it, off, 64);
    if (lane_id() >= off) {
      ip += a;
      it += b;
    }
  }
  const uint32_t wave = tid / 64, n_waves = (nth + 63) / 64;
  if (lane_id() == 63) {
    part[wave] = ip;
    part[nth + wave] = it;
  }
  __syncthreads();
  if (tid == 0)
    for (uint32_t w = 1; w < n_waves; ++w) {
      part[w] += part[w - 1];
      part[nth + w] += part[nth + w - 1];
    }
  __syncthreads();
  if (wave > 0) {
    ip += part[wave - 1];
    it += part[nth + wave - 1];
  }
  uint32_t op = ip - sp, ot = it - st;
  for (uint32_t e = e0; e < e1; ++e) {
    const uint32_t c = cnt[e];
    const uint32_t nt = (c + kGTok - 1) / kGTok;
    cnt[e] = op;
    tcnt[e] = ot;
    for (uint32_t j = 0; j < nt; ++j) {
      GroupTile t;
      t.blob = reinterpret_cast<const uint8_t *>(p.table[e]);
      t.start = op + j * kGTok;
      t.count = min(kGTok, c - j * kGTok);
      p.tiles[ot + j] = t;
    }
    op += c;
    ot += nt;
  }
  if (tid == nth - 1) *p.n_tiles = it;
  __syncthreads();
  for (uint32_t q = tid; q < p.n_pairs; q += nth)
    if (pos[q] != 0xffffffffu) p.plist[cnt[pos[q] >> 16] + (pos[q] & 0xffffu)] = q;
}

// Stage one (16 RT)-row x (32 / RT)-block slab of weights into LDS: one
// two-block chunk per thread, loaded with raw buffer loads into a register
// buffer (a chunk past the row's end reads zeros) and stored as int8 rows
// plus f32 scales.
template <int FMT, int RT>
struct Stager {
  using Geo = GGeom<RT>;
  using T = FmtTraits<FMT>;
  static constexpr int kDw = T::kChunkDwords;
  __amdgpu_buffer_rsrc_t rsrc;           // one descriptor for the whole slab (uniform, so no per-lane waterfall)
  uint32_t voff;      // byte offset of this thread's chunk (stage 0)
  uint32_t schunk;
  uint32_t srow;
  using Buf = uint32_t[kDw];

  // fused: slab rows 0 .. 8 RT - 1 are gate rows starting at base, the
  // next 8 RT the same up rows, up_off bytes further; otherwise 16 RT
  // consecutive rows.
  __device__ __forceinline__ void init(const uint8_t *base, uint32_t up_off, uint32_t row_bytes, bool fused) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, 0x7fffffff, 0x00020000);
    const uint32_t c = threadIdx.x;  // chunk of the slab: row c / kStageChunks
    srow = c / Geo::kStageChunks;
    schunk = c % Geo::kStageChunks;
    const bool up = fused && srow >= Geo::kRows / 2;
    const uint32_t r = up ? srow - Geo::kRows / 2 : srow;
    voff = (up ? up_off : 0u) + r * row_bytes + schunk * (uint32_t)T::kChunkBytes;
  }

  // Issue the loads of stage s (its kStageChunks chunks of each row) into
  // w.  Chunks past the row's end (and every chunk of a stage past the
  // last) read zeros, so the loads are issued unconditionally: w is
  // redefined on every path, which keeps the register buffers in place
  // instead of merging two versions of them after a branch.
  __device__ __forceinline__ void load(uint32_t s, uint32_t row_chunks, Buf &w) const {
    const bool ok = s * Geo::kStageChunks + schunk < row_chunks;
    const uint32_t off = ok ? voff + s * Geo::kStageChunks * (uint32_t)T::kChunkBytes : kNoChunkG;
#pragma unroll
    for (int v = 0; v < kDw / 4; ++v) {
      const uint4 q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 16 * v, 0, 0));
      w[4 * v] = q.x;
      w[4 * v + 1] = q.y;
      w[4 * v + 2] = q.z;
      w[4 * v + 3] = q.w;
    }
    w[kDw - 1] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, off + 16 * (kDw / 4), 0, 0);
  }

  // Write the loaded chunks to LDS: q as int8 [row][block][32], scales
  // as f32 [block][row].
  __device__ __forceinline__ void store(const Buf &w, uint8_t *lq, float *ld) const {
    {
      uint32_t q0[8], q1[8];
      float d0, d1;
      if constexpr (FMT == FMT_Q4_0) {
        // block 0: d = w0[15:0], qs = bytes 2..17; block 1: d = w4[31:16], qs = w5..w8
        const uint32_t a[4] = {realign16(w[0], w[1]), realign16(w[1], w[2]), realign16(w[2], w[3]),
                               realign16(w[3], w[4])};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          // element j = low nibble of qs[j], j + 16 = high nibble; int8 q - 8
          q0[m] = ((a[m] & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
          q0[4 + m] = (((a[m] >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
          const uint32_t b = w[5 + m];
          q1[m] = ((b & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
          q1[4 + m] = (((b >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
        }
        d0 = f16_bits_to_f32(w[0] & 0xffffu);
        d1 = f16_bits_to_f32(w[4] >> 16);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          q0[k] = realign16(w[k], w[k + 1]);
          q1[k] = w[9 + k];
        }
        d0 = f16_bits_to_f32(w[0] & 0xffffu);
        d1 = f16_bits_to_f32(w[8] >> 16);
      }
      const uint32_t b0 = 2 * schunk;
      uint4 *dst = reinterpret_cast<uint4 *>(lq + srow * Geo::kRowStride + b0 * 32);
      dst[0] = make_uint4(q0[0], q0[1], q0[2], q0[3]);
      dst[1] = make_uint4(q0[4], q0[5], q0[6], q0[7]);
      dst[2] = make_uint4(q1[0], q1[1], q1[2], q1[3]);
      dst[3] = make_uint4(q1[4], q1[5], q1[6], q1[7]);
      ld[b0 * Geo::kScaleStride + srow] = d0;
      ld[(b0 + 1) * Geo::kScaleStride + srow] = d1;
    }
  }
};

// One workgroup (4 waves) per (token tile, 16 RT staged rows).  FUSED:
// rows 0 .. 8 RT - 1 are gate rows, the next 8 RT the same up rows; the
// epilogue writes h = silu(g) * u for 8 RT rows = RT / 4 blocks per pair.
// Otherwise 16 RT down rows; the epilogue writes w_i * y_i per pair.
template <int FMT, bool FUSED, int RT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kGWavesPerEu))) void gproj_kernel(GroupedParams p) {
  using Geo = GGeom<RT>;
  using SG = Stager<FMT, RT>;
  constexpr uint32_t kRows = Geo::kRows, kSB = Geo::kStageBlocks, kStride = Geo::kRowStride, kSS = Geo::kScaleStride;
  constexpr int kWB = Geo::kWaveBlocks;
  // Two LDS slabs: stage s + 1 is stored into one while stage s is read
  // from the other, so a stage needs one barrier.
  __shared__ __attribute__((aligned(16))) uint8_t lq_buf[2][kRows * kStride];
  __shared__ __attribute__((aligned(16))) float ld_buf[2][kSB * kSS];
  uint8_t *const lq = lq_buf[0];

  const uint32_t row_tiles = FUSED ? p.d_ff / (kRows / 2) : p.d_model / kRows;
  const uint32_t tile = blockIdx.x / row_tiles;
  const uint32_t rt = blockIdx.x % row_tiles;
  if (tile >= *p.n_tiles) return;  // uniform over the workgroup
  const GroupTile gt = p.tiles[tile];
  const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / 64u;
  // B operands: the lane's column is the tile's pair lane % 16; its k-group
  // is lane / 16.  Every lane reads its column's pair index (16 words per
  // wave) before the weights are issued: loads complete in issue order, so
  // the B addresses never wait for weights.
  const uint32_t col = lane % 16, kg = lane / 16;
  const uint32_t pair = col < gt.count ? p.plist[gt.start + col] : 0xffffffffu;
  const bool col_ok = pair != 0xffffffffu;

  const uint32_t kblocks = FUSED ? p.xblocks : p.hblocks;  // K / 32
  const uint32_t row_chunks = kblocks / 2;
  const uint32_t row_bytes = kblocks * (uint32_t)FmtTraits<FMT>::kBlockBytes;
  SG sg;
  if constexpr (FUSED) {
    sg.init(gt.blob + (size_t)rt * (kRows / 2) * row_bytes, (uint32_t)p.proj_bytes, row_bytes, true);
  } else {
    sg.init(gt.blob + 2 * p.proj_bytes + (size_t)rt * kRows * row_bytes, 0u, row_bytes, false);
  }
  const uint32_t n_stages = (kblocks + kSB - 1) / kSB;
  // Two register buffers of weight loads: W(s) lives in wbuf[s & 1].
  typename SG::Buf wbuf[2];
  sg.load(0, row_chunks, wbuf[0]);
  sg.load(1, row_chunks, wbuf[1]);
  __builtin_amdgcn_sched_barrier(0);  // the weights go out before anything waits for the pair index

  // the lane's record of block 0 (block b's is 4 records = 8 uint4 further):
  // one 32 x 32 -> 64-bit multiply of the vector index by the record stride
  const uint4 *vrec;
  {
    const uint32_t v = col_ok ? (FUSED ? pair / p.top_k : pair) : 0u;
    const uint32_t stride = (FUSED ? p.xblocks : p.hblocks) * 8u;
    vrec = reinterpret_cast<const uint4 *>(FUSED ? p.xg : p.hg) + ((uint64_t)v * stride + kg * 2u);
  }

  float acc[RT][4];
#pragma unroll
  for (int a = 0; a < RT; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[a][i] = 0.f;

  // B operands of this wave's blocks of stage s (wave, wave + 4, ...) live
  // in slot s & 1.  A lane without a valid block (or a stage past the last)
  // reads block 0 of its record and gets a zero scale.
  uint2 bv[2][kWB][3];
  float bs[2][kWB];
  bool bok[2][kWB];
  auto load_b = [&](uint32_t s, int slot) {
    const uint32_t left = s < n_stages ? kblocks - s * kSB : 0u;
#pragma unroll
    for (int j = 0; j < kWB; ++j) {
      const uint32_t b = wave + 4 * j;
      bok[slot][j] = col_ok && b < left;
      const uint32_t gb = bok[slot][j] ? s * kSB + b : 0u;
      const uint4 *rp = vrec + gb * 8u;
      const uint4 r0 = rp[0], r1 = rp[1];
      bv[slot][j][0] = make_uint2(r0.x, r0.y);
      bv[slot][j][1] = make_uint2(r0.z, r0.w);
      bv[slot][j][2] = make_uint2(r1.x, r1.y);
      bs[slot][j] = __uint_as_float(r1.z);
    }
  };
  // Loads and slabs alternate between two buffers: at round s the wave
  // issues B(s + 1) and W(s + 2), stores W(s + 1) into the slab stage s
  // does not read, computes stage s and meets the others at the barrier.
  // Every load and store is issued unconditionally (weights past the last
  // stage read zeros without touching memory; B operands past it re-read
  // block 0), so each register buffer is redefined on every path: no
  // branch merges two versions of a buffer, which the compiler would
  // resolve with copies that wait for the loads just issued.  The prologue
  // leaves the loads outstanding in the loop's order (W(s + 1) older than
  // B(s + 1), W(s + 2)), so the wait counts are the same on the first round
  // as on every later one.  (Measured, config 3 gate/up: one slab with two
  // barriers per stage 69 us, two slabs 61-63 us.)
  load_b(0, 0);
  __builtin_amdgcn_sched_barrier(0);  // B(0) issued before the wait for W(0)
  sg.store(wbuf[0], lq_buf[0], ld_buf[0]);
  __syncthreads();
  auto stage = [&](uint32_t s, int slot) {
    const uint8_t *sl = lq_buf[slot];
    const float *sd = ld_buf[slot];
    const uint32_t nb = min(kSB, kblocks - s * kSB);
#pragma unroll
    for (int j = 0; j < kWB; ++j) {
      const uint32_t b = wave + 4 * j;
      if (b >= nb) break;  // uniform
      const float bsj = bok[slot][j] ? bs[slot][j] : 0.f;
      long bk[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) bk[k] = (long)(((uint64_t)bv[slot][j][k].y << 32) | bv[slot][j][k].x);
#pragma unroll
      for (int a = 0; a < RT; ++a) {
        const long av = *reinterpret_cast<const long *>(sl + (a * 16 + col) * kStride + b * 32 + kg * 8);
        const v4i z = {0, 0, 0, 0};
        const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bk[0], z, 0, 0, 0);
        const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bk[1], z, 0, 0, 0);
        const v4i p2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bk[2], z, 0, 0, 0);
        const float4 d = *reinterpret_cast<const float4 *>(&sd[b * kSS + a * 16 + kg * 4]);
        const float dd[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float hi = (float)(p1[i] + (p2[i] << 8));
          const float v = __builtin_fmaf(hi, 256.0f, (float)p0[i]);
          acc[a][i] = __builtin_fmaf(v, dd[i] * bsj, acc[a][i]);
        }
      }
    }
  };
  for (uint32_t s = 0; s < n_stages; s += 2) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint32_t st = s + b;
      load_b(st + 1, b ^ 1);
      sg.load(st + 2, row_chunks, wbuf[b]);
      sg.store(wbuf[b ^ 1], lq_buf[b ^ 1], ld_buf[b ^ 1]);
      if (st < n_stages) stage(st, b);  // uniform
      __syncthreads();
    }
  }

  // Sum the four waves' partials (in the slabs' LDS, free now): wave w
  // then owns row tiles w, w + 4, ...
  constexpr int kOwn = RT / 4;
  typedef float RedT[RT][64][4];  // [row tile][lane][i]
  RedT *red = reinterpret_cast<RedT *>(lq);
  static_assert(sizeof(RedT) * 4 <= sizeof(lq_buf), "reduction fits in the slabs");
#pragma unroll
  for (int a = 0; a < RT; ++a)
    *reinterpret_cast<float4 *>(&red[wave][a][lane][0]) = make_float4(acc[a][0], acc[a][1], acc[a][2], acc[a][3]);
  __syncthreads();
  float4 sum[kOwn];
#pragma unroll
  for (int o = 0; o < kOwn; ++o) {
    sum[o] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // fixed order
      const float4 v = *reinterpret_cast<const float4 *>(&red[w][wave + 4 * o][lane][0]);
      sum[o].x += v.x;
      sum[o].y += v.y;
      sum[o].z += v.z;
      sum[o].w += v.w;
    }
  }
  // lane holds rows (wave + 4 o) * 16 + 4 * kg + i of column col

  if constexpr (FUSED) {
    __syncthreads();
    float *fin = reinterpret_cast<float *>(lq);  // [16 RT rows][16 cols]
#pragma unroll
    for (int o = 0; o < kOwn; ++o) {
      const uint32_t r = (wave + 4 * o) * 16 + 4 * kg;
      fin[(r + 0) * kGTok + col] = sum[o].x;
      fin[(r + 1) * kGTok + col] = sum[o].y;
      fin[(r + 2) * kGTok + col] = sum[o].z;
      fin[(r + 3) * kGTok + col] = sum[o].w;
    }
    __syncthreads();
    if (tid < 64 * kOwn) {
      // h block hk of the workgroup, pair column c, k-group m: h rows
      // 32 hk + 8m .. +7 (gate rows there, up rows 8 RT further)
      const uint32_t hk = tid / 64, c = (tid / 4) % 16, m = tid % 4;
      float h[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float g = fin[(32 * hk + 8 * m + i) * kGTok + c];
        const float u = fin[(kRows / 2 + 32 * hk + 8 * m + i) * kGTok + c];
        h[i] = silu_mul(g, u, p.swiglu_limit);
      }
      const uint32_t pr = __shfl(pair, (int)c, 64);  // lane c of every wave holds column c's pair
      const bool ok = pr != 0xffffffffu;
      const size_t hb = (size_t)(ok ? pr : 0) * p.hblocks + rt * kOwn + hk;
      quant_group(h, p.hg + (hb * 4 + m) * kGRec, ok, p.q8act != 0);
    }
  } else {
    if (col_ok) {
      const float w = p.weights ? p.weights[pair] : 1.0f;
#pragma unroll
      for (int o = 0; o < kOwn; ++o) {
        const uint32_t r = rt * kRows + (wave + 4 * o) * 16 + 4 * kg;
        *reinterpret_cast<float4 *>(p.partial + (size_t)pair * p.d_model + r) =
            make_float4(w * sum[o].x, w * sum[o].y, w * sum[o].z, w * sum[o].w);
      }
    }
  }
}

// out[t] = [x +] sum over the token's valid slots, in slot order, of the
// pair partials (w_i y_i).  One thread per 4 output elements; the slots'
// validity comes from the grouping kernel, so all loads are independent.
__global__ __launch_bounds__(256) void gcombine_kernel(GroupedParams p) {
  const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t per_tok = p.d_model / 4;
  if (q >= p.n_tok * per_tok) return;
  const uint32_t t = q / per_tok, c = (q % per_tok) * 4;
  // Slots are summed in slot order; the loads of up to eight slots are
  // issued before any is used, so the combine costs one memory round trip
  // per eight slots instead of one per slot.
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t k0 = 0; k0 < p.top_k; k0 += 8) {
    bool ok[8];
    float4 v[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) ok[j] = k0 + j < p.top_k && p.pair_ok[t * p.top_k + k0 + j];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j)
      v[j] = ok[j] ? *reinterpret_cast<const float4 *>(p.partial + (size_t)(t * p.top_k + k0 + j) * p.d_model + c)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j)
      if (ok[j]) {
        acc.x += v[j].x;
        acc.y += v[j].y;
        acc.z += v[j].z;
        acc.w += v[j].w;
      }
  }
  float4 *o = reinterpret_cast<float4 *>(p.out + (size_t)t * p.d_model + c);
  if (p.flags & (kFlagResidual | kFlagAccumulate)) {
    const float4 base = (p.flags & kFlagResidual) ? *reinterpret_cast<const float4 *>(p.x + (size_t)t * p.d_model + c)
                                                  : *o;
    acc = make_float4(base.x + acc.x, base.y + acc.y, base.z + acc.z, base.w + acc.w);
  }
  *o = acc;
}

}  // namespace

size_t grouped_group_lds_bytes(uint32_t table_len, uint32_t n_pairs) {
  return (size_t)(2 * table_len + n_pairs) * 4;
}

hipError_t launch_grouped_prep(const GroupedParams &p, hipStream_t st) {
  const uint32_t quads = p.n_tok * p.xblocks * 4;
  const uint32_t gblocks = 1 + (quads + 1023) / 1024;
  hipLaunchKernelGGL(group_kernel, dim3(gblocks), dim3(1024), grouped_group_lds_bytes(p.table_len, p.n_pairs), st, p);
  return hipGetLastError();
}

hipError_t launch_grouped_proj(int fmt, bool fused, const GroupedParams &p, uint32_t max_tiles, hipStream_t st) {
  // Down runs 128-row workgroups (RT = 8) wherever d_model divides by 128.
  // Gate/up does so (64 gate + 64 up rows) only from 2048 routed pairs on:
  // with fewer its launch fills too few rounds of the resident workgroup
  // slots.  Measured on the Qwen3 Q8_0 shape, gate/up us at RT = 4 / 8:
  // 16 tokens 36.7 / 41.1, 64 tokens 62.2 / 69.2, 128 tokens 89.2 / 92.1,
  // 256 tokens 144.6 / 136.4; down at 64 tokens 38.9 -> 36.1, at 256
  // tokens 94 -> 75.
  const bool wide = fused ? (p.d_ff % 64 == 0 && p.n_pairs >= 2048) : p.d_model % 128 == 0;
  const uint32_t rows = wide ? 128 : 64;
  const uint32_t grid = max_tiles * (fused ? p.d_ff / (rows / 2) : p.d_model / rows);
#define MER_GPROJ(F, FU, R) hipLaunchKernelGGL((gproj_kernel<F, FU, R>), dim3(grid), dim3(256), 0, st, p)
  if (fmt == FMT_Q4_0) {
    if (fused && wide) MER_GPROJ(FMT_Q4_0, true, 8);
    else if (fused) MER_GPROJ(FMT_Q4_0, true, 4);
    else if (wide) MER_GPROJ(FMT_Q4_0, false, 8);
    else MER_GPROJ(FMT_Q4_0, false, 4);
  } else {
    if (fused && wide) MER_GPROJ(FMT_Q8_0, true, 8);
    else if (fused) MER_GPROJ(FMT_Q8_0, true, 4);
    else if (wide) MER_GPROJ(FMT_Q8_0, false, 8);
    else MER_GPROJ(FMT_Q8_0, false, 4);
  }
#undef MER_GPROJ
  return hipGetLastError();
}

hipError_t launch_grouped_combine(const GroupedParams &p, hipStream_t st) {
  const uint32_t cq = p.n_tok * (p.d_model / 4);
  hipLaunchKernelGGL(gcombine_kernel, dim3((cq + 255) / 256), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace mer
