// mer_internal.hpp -- shared declarations between the kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mer_device.hpp"

namespace mer {

// Rows per pass of one lane group: the fused gate/up walk streams 2 rows
// of each projection per pass (4 chunks in flight per lane), the down walk
// streams 4 rows.
constexpr int kFusedRows = 2;
constexpr int kDownRows = 4;
// Chunks a lane may keep register-resident in the fused gate/up walk.
constexpr int max_fused_cpl(int fmt) { return fmt == FMT_Q4_0 ? 2 : 1; }

// Arguments of one projection launch (passed by value).
struct ProjParams {
  const void *const *table;  // expert table (device), or null with `single`
  uint32_t table_len;
  const int32_t *ids;        // instance -> expert id (device)
  const uint8_t *single;     // single expert blob (device), overrides table
  uint32_t n_inst;           // expert instances (token x slot)
  size_t proj_off0;          // byte offset of the (gate | down) projection
  size_t proj_off1;          // byte offset of the up projection (fused)
  uint32_t rows;             // output rows of the projection
  uint32_t chunks;           // 64-weight chunks per row
  uint32_t slices;           // column slices
  uint32_t chunks_per_slice;
  uint32_t waves_per_slice;  // waves walking one (instance, slice)
  uint32_t rows_per_wave;
  const float *x;            // input vectors
  uint32_t x_div;            // input index = instance / x_div
  size_t x_stride;           // floats between consecutive inputs
  float *out;                // [n_inst][slices][rows]
};

struct ProjPlan {
  bool fast;
  int G, CPL;
  uint32_t slices, chunks_per_slice, waves_per_slice, rows_per_wave;
};

struct CombineParams {
  const float *partial;  // [n_tokens*top_k][slices][d_model]
  const float *weights;  // [n_tokens*top_k] or null (weight 1, no skip)
  const float *x;        // residual input
  float *out;
  uint32_t n_tokens, top_k, slices, d_model;
  uint32_t flags;
};

hipError_t launch_proj(int fmt, bool fused, const ProjPlan &plan, const ProjParams &p, hipStream_t st);
hipError_t launch_generic(int fmt, bool fused, const ProjParams &p, uint32_t cols, hipStream_t st);
hipError_t launch_combine(const CombineParams &c, hipStream_t st);
hipError_t launch_dequant(int fmt, const uint8_t *src, size_t n_weights, float *dst, hipStream_t st);
hipError_t launch_q4_raw(const uint8_t *w, size_t w_block_off, uint32_t rows, uint32_t bpr,
                         const float *x, float *y, hipStream_t st);
hipError_t launch_fill(int fmt, uint64_t seed, uint64_t expert, uint64_t block_begin, uint64_t n_blocks,
                       float lo, float hi, uint8_t *dst, hipStream_t st);
hipError_t read_and_clear_device_status(uint32_t *out);

}  // namespace mer
