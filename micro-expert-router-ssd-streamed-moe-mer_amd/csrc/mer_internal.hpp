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
// Chunks a lane walks per row (G = 64); inputs beyond one chunk are read
// from LDS per pass.
constexpr int kMaxCpl = 4;

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
  uint32_t wgs_per_slice;    // workgroups walking one (instance, slice)
  uint32_t rows_per_wave;    // rows of one wave (a workgroup owns 4x)
  uint32_t lds_blocks;       // input blocks staged in LDS per workgroup
  const float *x;            // f32 input vectors (gate/up; generic kernel)
  uint32_t x_div;            // input index = instance / x_div
  size_t x_stride;           // floats between consecutive inputs
  const uint32_t *xq_dig;    // packed inputs of the down projection
  const float *xq_scale;     //   [n_inst][xq_blocks] digit planes / scales
  uint32_t xq_blocks;
  uint32_t *hq_dig;          // packed h written by the gate/up kernel
  float *hq_scale;           //   [n_inst][hq_blocks]
  uint32_t hq_blocks;
  float *out;                // down: [n_inst][slices][rows]; gate/up: f32 h or null
};

inline size_t proj_lds_bytes(const ProjParams &p, bool fused) {
  return (size_t)p.lds_blocks * (kBlockDigitDwords * 4 + 4) + (fused ? (size_t)4 * p.rows_per_wave * 4 : 0);
}

struct ProjPlan {
  bool fast;
  int G, CPL;
  uint32_t slices, chunks_per_slice, wgs_per_slice, rows_per_wave;
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
