// mer_internal.hpp -- shared declarations between the kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mer_device.hpp"

namespace mer {

// A projection workgroup owns a tile of 32 output rows (one block of h for
// the gate/up kernel), 8 rows per wave.
constexpr uint32_t kRowsPerWave = 8;
constexpr uint32_t kTileRows = 4 * kRowsPerWave;
constexpr int kMaxCpl = 4;

// prep_kernel: pack x per token, resolve one blob pointer per expert slot.
struct PrepParams {
  const void *const *table;  // expert table (device), or null with `single`
  uint32_t table_len;
  const int32_t *ids;        // [n_tokens * top_k]
  const float *weights;      // [n_tokens * top_k] slot weights, or null
  const uint8_t *single;     // single expert blob (overrides table / ids)
  uint32_t top_k;
  const uint8_t **inst_ptr;  // out: [n_tokens * top_k]
  const float *x;            // [n_tokens][d_model]
  uint32_t d_model;
  uint32_t blocks;           // d_model / 32
  uint32_t *xq_dig;          // out (fast path): [n_tokens][blocks][24], or null
  float *xq_scale;           // out: [n_tokens][blocks]
};

// Arguments of one projection launch (passed by value).
struct ProjParams {
  const uint8_t *const *inst_ptr;  // blob per expert instance (null = miss)
  uint32_t n_inst;
  size_t proj_off0;          // byte offset of the (gate | down) projection
  size_t proj_off1;          // byte offset of the up projection (fused)
  uint32_t rows;             // output rows of the projection
  uint32_t chunks;           // 64-weight chunks per row
  uint32_t slices;           // column slices
  uint32_t chunks_per_slice;
  uint32_t tiles;            // 32-row tiles per (instance, slice)
  const uint32_t *xq_dig;    // packed input vectors [.][xq_blocks][24]
  const float *xq_scale;     //   and their block scales
  uint32_t xq_blocks;
  uint32_t x_div;            // input index = instance / x_div
  uint32_t *hq_dig;          // gate/up: packed h [n_inst][hq_blocks][24]
  float *hq_scale;
  uint32_t hq_blocks;
  float *out;                // down: [n_inst][slices][rows]; gate/up: f32 h or null
  float swiglu_limit;        // gate clamp before SiLU (+inf = none)
};

// Flat-layout fallback (any shape): f32 inputs and outputs.
struct GenericParams {
  const uint8_t *const *inst_ptr;
  uint32_t n_inst;
  size_t proj_off0, proj_off1;
  uint32_t rows, cols;
  int fused;
  const float *x;
  uint32_t x_div;
  size_t x_stride;
  float *out;  // [n_inst][rows]
  float swiglu_limit;  // gate clamp before SiLU (+inf = none)
};

struct ProjPlan {
  bool fast;
  int G, CPL;
  uint32_t slices, chunks_per_slice, tiles;
};

struct CombineParams {
  const float *partial;  // [n_tokens*top_k][slices][d_model]
  const float *weights;  // [n_tokens*top_k] or null (weight 1, no skip)
  const float *x;        // residual input
  float *out;
  uint32_t n_tokens, top_k, slices, d_model;
  uint32_t flags;
};

// ---- persistent decode kernel (mer_decode.hip) -------------------------
constexpr uint32_t kFlagResidual = 1u;    // out = x + sum_i w_i y_i
constexpr uint32_t kFlagAccumulate = 2u;  // out += sum_i w_i y_i
constexpr uint32_t kFlagChain = 4u;       // layer l > 0 reads layer l-1's out
constexpr uint32_t kFlagRouteAfterPrev = 8u;  // layer l > 0 touches its experts after layer l-1 completes
constexpr uint32_t kFlagQ8Act = 16u;  // Q4_0: activations quantised to Q8_0 as Candle's QMatMul does
constexpr uint32_t kMaxLayers = 64;
constexpr uint32_t kLineDwords = 32;     // decode digit block: 24 digit dwords, scale, padding
constexpr uint32_t kPollStride = 64;     // words between polled decode counters (one 256-byte line each)
constexpr uint32_t kFlagStride = 32;     // 64-bit release flags between polled flags (one 256-byte line each)
constexpr uint32_t kReleaseFan = 16;     // release flags per (layer, token), one line each
constexpr uint32_t kCombineBatch = 16;   // partial sums a decode combine loads in one batch
// Control lines of a decode workspace (one 256-byte line each): exit count,
// abort flag, kExitGroups exit-group counters, then the launch epoch word.
// Waves leave through a two-level count (a group counter, then the exit
// count for the last wave of each group): device-scope atomics on one
// address are serialised, ~20 ns each, so 3072 exits on one counter would
// take ~60 us.
constexpr uint32_t kExitGroups = 64;
constexpr uint32_t kCtlEpochLine = 2 + kExitGroups;
constexpr uint32_t kCtlLines = 3 + kExitGroups;

struct LayerArgs {
  const void *const *table;  // device array of expert blob pointers
  uint32_t table_len;
  const int32_t *ids;        // [n_tok * top_k]
  const float *weights;      // [n_tok * top_k] or null (weight 1, no skip)
  const float *x;            // [n_tok][d_model] (layer 0, or every layer without chaining)
  float *out;                // [n_tok][d_model]
};

struct DecodeParams {
  LayerArgs layers[kMaxLayers];
  const uint8_t *single;     // single-expert mode: this blob for every slot
  uint32_t n_layers, n_tok, top_k, n_inst;
  uint32_t d_model, d_ff, flags;
  float swiglu_limit;        // gate clamp before SiLU (+inf = none)
  size_t proj_bytes;         // bytes of one projection
  uint32_t xblocks, hblocks; // d_model / 32, d_ff / 32
  uint32_t g_chunks, g_slices, g_cps, g_tiles;  // gate/up: chunks per row, slices, chunks per slice, tiles
  uint32_t d_chunks, d_slices, d_cps, d_tiles;  // down
  uint32_t p_items;          // packing items per token
  uint32_t combine_packs;    // layer l > 0's input is packed by layer l-1's combines (P items idle)
  uint32_t items_per_layer, off_p, off_g, off_d;
  uint64_t total_items;
  // scratch, all [layer]-major
  // The launch's epoch is read from *epoch_word at entry by every wave; the
  // last wave out stores a fresh value, unique on the device, for the next
  // launch on this workspace (so a replayed HIP graph gets a new epoch too).
  // Epochs tag digit lines and release flags; 0 is never an epoch.
  uint64_t *epoch_word;
  // Digit planes in the decode kernel's line format: one 128-byte line per
  // 32-element block, digit dwords 0..23, the f32 block scale in dword 24 and
  // the 64-bit epoch of the launch that wrote it in dwords 25..26.
  uint32_t *xq_dig;          // [L][n_tok][xblocks][32]
  uint32_t *hq_dig;          // [L][n_inst][hblocks][32]
  float *gpart;              // [L][n_inst][g_slices][2][d_ff]  (g_slices > 1)
  float *partial;            // [L][n_inst][d_slices][d_model]
  uint32_t *counters;        // [L][cnt_per_layer], zero between launches
  uint32_t cnt_per_layer, c_p, c_ga, c_gd, c_da, c_c;
  uint32_t n_counters;
  uint64_t *release;         // [L][n_tok][kReleaseFan] epoch flags (never cleared: other epochs read as not set)
  uint64_t *gd_release;      // [L][n_inst][d_slices][kReleaseFan] h-slice release flags, or null (counters)
  uint32_t *exit_count;
  uint32_t *exit_groups;      // kExitGroups counters, kPollStride words apart
  uint32_t *abort_flag;      // set by a timed-out wait; later waits give up
  uint32_t *status;
  uint64_t timeout_ticks;
  uint64_t *trace;           // optional item trace [trace_cap][4], or null
  uint64_t trace_cap;
};

// ---- grouped multi-token path (mer_grouped.hip) --------------------------
constexpr uint32_t kMaxGroupedExperts = 4096;  // table entries the grouping kernel counts in LDS
constexpr uint32_t kMaxGroupedPairs = 4096;    // routed (token, slot) pairs per call

struct GroupTile {
  const uint8_t *blob;  // the expert's blob
  uint32_t start;       // first pair of the tile in plist
  uint32_t count;       // pairs in the tile (1..16)
};

struct GroupedParams {
  const void *const *table;
  uint32_t table_len;
  const int32_t *ids;        // [n_tok * top_k]
  const float *weights;      // [n_tok * top_k] or null (weight 1, no skip)
  const float *x;            // [n_tok][d_model]
  float *out;                // [n_tok][d_model]
  uint32_t flags;
  uint32_t q8act;            // Q4_0 under MER_MOE_QMM: inputs quantised as Candle's Q8_0
  uint32_t n_tok, top_k, n_pairs;
  uint32_t d_model, d_ff, xblocks, hblocks;
  float swiglu_limit;        // gate clamp before SiLU (+inf = none)
  size_t proj_bytes;
  // scratch
  uint32_t *xg;              // x digit records [n_tok][xblocks][4 k-groups][8 dwords]
  uint32_t *hg;              // h digit records [n_pairs][hblocks][4][8 dwords]
  float *partial;            // w_i y_i [n_pairs][d_model]
  uint32_t *plist;           // pairs grouped by expert [n_pairs]
  uint32_t *pair_ok;         // [n_pairs] 1 = routed to a resident expert with a nonzero weight
  GroupTile *tiles;          // [max tiles]
  uint32_t *n_tiles;         // tiles emitted by the grouping kernel
  uint32_t *status;
};

size_t grouped_group_lds_bytes(uint32_t table_len, uint32_t n_pairs);
hipError_t launch_grouped_prep(const GroupedParams &p, hipStream_t st);
hipError_t launch_grouped_proj(int fmt, bool fused, const GroupedParams &p, uint32_t max_tiles, hipStream_t st);
hipError_t launch_grouped_combine(const GroupedParams &p, hipStream_t st);

// ---- LinearGate router (mer_router.hip) -----------------------------------
constexpr uint32_t kMaxRouterExperts = 1024;
constexpr uint32_t kMaxRouterTopK = 64;
constexpr uint32_t kMaxRouterGroups = 64;

struct RouterParams {
  const float *gate;    // [n_experts][d_model]
  const float *x;       // [n_tokens][d_model]
  const float *bias;    // [n_experts] selection-only correction bias, or null
  int32_t *ids;         // [n_tokens][top_k]; -1 where fewer experts qualify
  float *weights;       // [n_tokens][top_k]; 0 where fewer experts qualify
  float *logits;        // [n_tokens][n_experts], or null
  float *logit_buf;     // [n_tokens][n_experts]: logits, or the library's buffer when logits is null
  uint32_t n_experts, d_model, n_tokens, top_k;
  int32_t scoring;      // 0 softmax, 1 sigmoid
  int32_t normalise;    // renormalise the top-k weights
  uint32_t n_group, topk_group;
  float scaling;        // routed scaling factor
};

hipError_t launch_router(const RouterParams &p, hipStream_t st);

const void *decode_kernel_fn(int fmt, int gg, int gd, bool pair, bool q8act);
hipError_t launch_decode(const void *fn, uint32_t grid, uint32_t waves_per_group, const DecodeParams &p,
                         hipStream_t st);
uint32_t *device_status_ptr();
hipError_t launch_decode_scratch_prep(uint32_t *ctl, uint32_t n_ctl, uint32_t *zero, size_t n_zero,
                                      uint64_t *epoch_word, hipStream_t st);

hipError_t launch_prep(int fmt, const PrepParams &q, uint32_t n_tokens, hipStream_t st);
hipError_t launch_proj(int fmt, bool fused, const ProjPlan &plan, const ProjParams &p, hipStream_t st);
hipError_t launch_generic(int fmt, const GenericParams &p, hipStream_t st);
hipError_t launch_combine(const CombineParams &c, hipStream_t st);
hipError_t launch_dequant(int fmt, const uint8_t *src, size_t n_weights, float *dst, hipStream_t st);
hipError_t launch_q4_raw(const uint8_t *w, size_t w_block_off, uint32_t rows, uint32_t bpr,
                         const float *x, float *y, hipStream_t st);
hipError_t launch_fill(int fmt, uint64_t seed, uint64_t expert, uint64_t block_begin, uint64_t n_blocks,
                       float lo, float hi, uint8_t *dst, hipStream_t st);
hipError_t launch_f16_in(const uint16_t *x, size_t d_model, size_t n_rep, float *dst, hipStream_t st);
hipError_t launch_f16_out(const float *src, size_t n, uint16_t *dst, hipStream_t st);
hipError_t launch_zero(float *dst, size_t n, hipStream_t st);
hipError_t read_and_clear_device_status(uint32_t *out);

// Error reporting shared by the C-ABI sources: record `msg` (and a HIP
// error's text) as the calling thread's last error and return `status`.
int report_error(int status, const char *msg);
int report_hip_error(hipError_t e, int status, const char *what);
// MER_OK once mer_hip_init has selected a device.
int check_initialised();

}  // namespace mer
