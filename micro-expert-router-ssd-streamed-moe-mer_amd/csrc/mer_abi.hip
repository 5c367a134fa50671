// mer_abi.hip -- extern "C" boundary of the routed-expert SwiGLU FFN
// (declared in include/mer_hip.h).  Host-side validation mirrors the
// reference's typed errors; device work is enqueued on the caller's stream.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/mer_hip.h"
#include "mer_internal.hpp"

using namespace mer;

namespace {

thread_local std::string t_err;
thread_local mer_error_info t_info;

int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_err = buf;
  t_info = mer_error_info{status, 0, 0, 0, 0};
  return status;
}

int fail_size(int status, size_t have, size_t need, size_t dm, size_t dff) {
  char buf[256];
  if (status == MER_ERR_TRUNCATED_PAYLOAD)
    snprintf(buf, sizeof buf,
             "expert payload truncated: have %zu bytes, need %zu for d_model=%zu, d_ff=%zu "
             "(shortfall %zu bytes)",
             have, need, dm, dff, need - have);
  else
    snprintf(buf, sizeof buf, "expert buffer too small: have %zu bytes, need %zu for d_model=%zu, d_ff=%zu",
             have, need, dm, dff);
  t_err = buf;
  t_info = mer_error_info{status, have, need, dm, dff};
  return status;
}

int ok() { return MER_OK; }

// EXPERT_SIZE_TOLERANCE_BYTES = DEFAULT_BLOCK_ALIGN (inference.rs:3962).
constexpr size_t kTolerance = 4096;

size_t sat_mul(size_t a, size_t b) { return (a != 0 && b > SIZE_MAX / a) ? SIZE_MAX : a * b; }
bool checked_mul(size_t a, size_t b, size_t *o) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *o = a * b;
  return true;
}
size_t div_ceil(size_t a, size_t b) { return a / b + (a % b != 0); }
size_t block_bytes(int dtype) { return dtype == MER_DTYPE_Q4_0 ? 18 : 34; }
int fmt_of(int dtype) { return dtype == MER_DTYPE_Q4_0 ? FMT_Q4_0 : FMT_Q8_0; }

struct DeviceState {
  bool ready = false;
  int cus = 256;
  uint32_t waves_per_cu = 12;
  float *scratch = nullptr;
  size_t scratch_floats = 0;
};
std::mutex g_mu;
int g_device = -1;
DeviceState g_dev[64];

// GPU stage timings (stage_timing.rs:6-29 analogue): when enabled, every
// gate/up, down and combine launch is bracketed by a pair of events on the
// launch stream; mer_hip_stage_timing_read sums their elapsed times.
enum Stage { STAGE_GATE_UP = 0, STAGE_DOWN = 1, STAGE_COMBINE = 2, STAGE_COUNT = 3 };
struct TimedLaunch {
  hipEvent_t start, end;
  int stage;
};
bool g_timing = false;
std::vector<TimedLaunch> g_timed;
size_t g_timed_used = 0;

int timing_begin(int stage, hipStream_t st, TimedLaunch **slot) {
  *slot = nullptr;
  if (!g_timing) return MER_OK;
  if (g_timed_used == g_timed.size()) {
    TimedLaunch t{};
    if (hipEventCreate(&t.start) != hipSuccess || hipEventCreate(&t.end) != hipSuccess)
      return fail(MER_ERR_RUNTIME_INVARIANT, "stage timing event creation failed");
    g_timed.push_back(t);
  }
  TimedLaunch *t = &g_timed[g_timed_used++];
  t->stage = stage;
  hipError_t e = hipEventRecord(t->start, st);
  if (e != hipSuccess) return fail(MER_ERR_SUBMISSION, "stage timing record: %s", hipGetErrorString(e));
  *slot = t;
  return MER_OK;
}

int timing_end(TimedLaunch *t, hipStream_t st) {
  if (!t) return MER_OK;
  hipError_t e = hipEventRecord(t->end, st);
  if (e != hipSuccess) return fail(MER_ERR_SUBMISSION, "stage timing record: %s", hipGetErrorString(e));
  return MER_OK;
}

int require_init() {
  if (g_device < 0) return fail(MER_ERR_NOT_INITIALIZED, "mer_hip_init has not been called");
  return MER_OK;
}

int hip_fail(hipError_t e, int status, const char *what) {
  return fail(status, "%s: %s", what, hipGetErrorString(e));
}

// Grow the per-device scratch (h vectors and down-projection partials).
int ensure_scratch(size_t floats, float **out) {
  DeviceState &d = g_dev[g_device];
  if (d.scratch_floats < floats) {
    if (d.scratch) {
      hipError_t e = hipDeviceSynchronize();
      if (e != hipSuccess) return hip_fail(e, MER_ERR_DEVICE_LOST, "synchronise before scratch growth");
      (void)hipFree(d.scratch);
      d.scratch = nullptr;
      d.scratch_floats = 0;
    }
    size_t want = floats < (1u << 20) ? (1u << 20) : floats;
    hipError_t e = hipMalloc(&d.scratch, want * sizeof(float));
    if (e != hipSuccess) return hip_fail(e, MER_ERR_PHYSICAL_CAPACITY, "scratch allocation");
    d.scratch_floats = want;
  }
  *out = d.scratch;
  return MER_OK;
}

// Choose the decomposition of one projection launch.  `waves_per_cu`
// sets the grid size (default 12, MER_WAVES_PER_CU overrides at init).
ProjPlan plan_projection(size_t rows, size_t cols, uint32_t n_inst, bool fused, bool aligned) {
  ProjPlan pl{};
  // Fast path: rows of an even number of blocks (4-byte aligned chunks) and
  // 32-row blocks of h; every configuration of the benchmark qualifies.
  pl.fast = aligned && cols % 64 == 0 && rows % 64 == 0 && cols <= MER_MAX_EXPERT_DIM &&
            rows <= MER_MAX_EXPERT_DIM && rows > 0;
  if (!pl.fast) return pl;
  const uint32_t C = (uint32_t)(cols / 64);
  if (C <= 16) { pl.G = 16; pl.CPL = 1; pl.slices = 1; }
  else if (C <= 32) { pl.G = 32; pl.CPL = 1; pl.slices = 1; }
  else if (fused) { pl.G = 64; pl.CPL = (int)div_ceil(C, 64); pl.slices = 1; }
  else { pl.G = 64; pl.CPL = 1; pl.slices = (uint32_t)div_ceil(C, 64); }
  pl.chunks_per_slice = (uint32_t)div_ceil(C, pl.slices);
  const uint32_t R = fused ? kFusedRows : kDownRows;
  // rows of a wave: whole passes of all lane groups, and (gate/up) whole
  // 32-row blocks of h per 4-wave workgroup
  uint32_t unit = R * (64u / (uint32_t)pl.G);
  while (unit % 8) unit *= 2;
  const uint64_t target_waves = (uint64_t)g_dev[g_device].cus * g_dev[g_device].waves_per_cu;
  const uint64_t per_slice = (uint64_t)n_inst * pl.slices;
  uint64_t want = target_waves / per_slice;
  if (want < 4) want = 4;
  uint64_t rpw = div_ceil(rows, want);
  rpw = div_ceil(rpw, unit) * unit;
  pl.rows_per_wave = (uint32_t)rpw;
  pl.wgs_per_slice = (uint32_t)div_ceil(rows, 4 * rpw);
  return pl;
}

int validate(int dtype, size_t len, size_t x_len, size_t y_len, size_t dm, size_t dff, size_t tolerance) {
  if (dtype == MER_DTYPE_Q4_0) {
    // from_bytes_q4_0_with_tolerance (inference.rs:1766-1783, :4035-4077)
    size_t blocks = div_ceil(sat_mul(dff, dm), 32);
    size_t need = sat_mul(sat_mul(blocks, 3), 18);
    if (len < need) {
      if (need > kTolerance && need - len <= kTolerance) {
        if (need - len > tolerance) return fail_size(MER_ERR_TRUNCATED_PAYLOAD, len, need, dm, dff);
        return fail(MER_ERR_INVALID_LAYOUT,
                    "zero-padding a truncated payload is a host-side legacy mode; the device path is strict");
      }
      return fail_size(MER_ERR_BUFFER_TOO_SMALL, len, need, dm, dff);
    }
    // forward_candle builds x as a [d_model, 1] tensor (inference.rs:1460)
    if (x_len != dm) return fail(MER_ERR_COMPUTE, "shape mismatch: x has %zu values, d_model=%zu", x_len, dm);
    if (y_len < dm) return fail(MER_ERR_COMPUTE, "output holds %zu values, d_model=%zu", y_len, dm);
    return MER_OK;
  }
  if (dtype == MER_DTYPE_Q8_0) {
    // validate_q8_direct_layout (inference.rs:3349-3418)
    if (dm == 0 || dff == 0)
      return fail(MER_ERR_INVALID_LAYOUT, "Q8_0 dimensions must be non-zero, got d_model=%zu, d_ff=%zu", dm, dff);
    if (x_len != dm || y_len != dm)
      return fail(MER_ERR_INVALID_LAYOUT, "Q8_0 activation dimensions mismatch: x=%zu, y=%zu, d_model=%zu", x_len,
                  y_len, dm);
    size_t weights, proj, need;
    if (!checked_mul(dm, dff, &weights)) return fail(MER_ERR_INVALID_LAYOUT, "Q8_0 projection element count overflow");
    if (!checked_mul(div_ceil(weights, 32), 34, &proj)) return fail(MER_ERR_INVALID_LAYOUT, "Q8_0 projection byte count overflow");
    if (!checked_mul(proj, 3, &need)) return fail(MER_ERR_INVALID_LAYOUT, "Q8_0 expert byte count overflow");
    if (len < need) {
      if (need > kTolerance && need - len <= kTolerance) return fail_size(MER_ERR_TRUNCATED_PAYLOAD, len, need, dm, dff);
      return fail_size(MER_ERR_BUFFER_TOO_SMALL, len, need, dm, dff);
    }
    return MER_OK;
  }
  return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d (only Q4_0=4 and Q8_0=5)", dtype);
}

// Enqueue gate/up -> down -> combine for n_inst expert instances.
int run_experts(int dtype, size_t dm, size_t dff, uint32_t n_tokens, uint32_t top_k, const void *const *table,
                uint32_t table_len, const int32_t *ids, const uint8_t *single, const float *weights,
                const float *x, float *out, unsigned flags, hipStream_t st, bool direct_out) {
  const int fmt = fmt_of(dtype);
  const uint32_t n_inst = n_tokens * top_k;
  const size_t proj = div_ceil(dm * dff, 32) * block_bytes(dtype);
  const bool aligned = single ? ((uintptr_t)single % 4 == 0) : true;

  ProjPlan pg = plan_projection(dff, dm, n_inst, true, aligned);
  ProjPlan pd = plan_projection(dm, dff, n_inst, false, aligned);
  const bool fast = pg.fast && pd.fast;
  const uint32_t slices = fast ? pd.slices : 1;

  const bool write_direct = direct_out && slices == 1 && n_inst == 1 && flags == 0;
  // scratch: f32 h (generic path) | h digit planes + scales (fast path) | partials
  const size_t hblocks = dff / 32;
  const size_t h_floats = fast ? 0 : (size_t)n_inst * dff;
  const size_t hq_dwords = fast ? (size_t)n_inst * hblocks * kBlockDigitDwords : 0;
  const size_t hs_floats = fast ? (size_t)n_inst * hblocks : 0;
  const size_t p_floats = write_direct ? 0 : (size_t)n_inst * slices * dm;
  auto up64 = [](size_t v) { return (v + 63) / 64 * 64; };
  float *scratch = nullptr;
  int rc = ensure_scratch(up64(h_floats) + up64(hq_dwords) + up64(hs_floats) + up64(p_floats), &scratch);
  if (rc) return rc;
  float *h = scratch;
  uint32_t *hq_dig = reinterpret_cast<uint32_t *>(scratch + up64(h_floats));
  float *hq_scale = scratch + up64(h_floats) + up64(hq_dwords);
  float *partial = write_direct ? out : hq_scale + up64(hs_floats);

  ProjParams p{};
  p.table = table;
  p.table_len = table_len;
  p.ids = ids;
  p.single = single;
  p.n_inst = n_inst;

  // gate/up + SiLU -> h (digit planes on the fast path)
  p.proj_off0 = 0;
  p.proj_off1 = proj;
  p.rows = (uint32_t)dff;
  p.chunks = (uint32_t)(dm / 64);
  p.x = x;
  p.x_div = top_k;
  p.x_stride = dm;
  p.hq_dig = hq_dig;
  p.hq_scale = hq_scale;
  p.hq_blocks = (uint32_t)hblocks;
  hipError_t e;
  TimedLaunch *tl = nullptr;
  int trc = timing_begin(STAGE_GATE_UP, st, &tl);
  if (trc) return trc;
  if (fast) {
    p.out = nullptr;
    p.slices = 1;
    p.chunks_per_slice = pg.chunks_per_slice;
    p.wgs_per_slice = pg.wgs_per_slice;
    p.rows_per_wave = pg.rows_per_wave;
    p.lds_blocks = 2 * pg.chunks_per_slice;
    e = launch_proj(fmt, true, pg, p, st);
  } else {
    p.out = h;
    p.slices = 1;
    e = launch_generic(fmt, true, p, (uint32_t)dm, st);
  }
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "gate/up launch");
  if ((trc = timing_end(tl, st))) return trc;

  // down -> partial [inst][slice][dm]
  p.proj_off0 = 2 * proj;
  p.proj_off1 = 0;
  p.rows = (uint32_t)dm;
  p.chunks = (uint32_t)(dff / 64);
  p.x = h;
  p.x_div = 1;
  p.x_stride = dff;
  p.xq_dig = hq_dig;
  p.xq_scale = hq_scale;
  p.xq_blocks = (uint32_t)hblocks;
  p.out = partial;
  if ((trc = timing_begin(STAGE_DOWN, st, &tl))) return trc;
  if (fast) {
    p.slices = pd.slices;
    p.chunks_per_slice = pd.chunks_per_slice;
    p.wgs_per_slice = pd.wgs_per_slice;
    p.rows_per_wave = pd.rows_per_wave;
    p.lds_blocks = 2 * pd.chunks_per_slice;
    e = launch_proj(fmt, false, pd, p, st);
  } else {
    p.slices = 1;
    e = launch_generic(fmt, false, p, (uint32_t)dff, st);
  }
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "down launch");
  if ((trc = timing_end(tl, st))) return trc;
  if (write_direct) return MER_OK;

  CombineParams c{};
  c.partial = partial;
  c.weights = weights;
  c.x = x;
  c.out = out;
  c.n_tokens = n_tokens;
  c.top_k = top_k;
  c.slices = slices;
  c.d_model = (uint32_t)dm;
  c.flags = flags;
  if ((trc = timing_begin(STAGE_COMBINE, st, &tl))) return trc;
  e = launch_combine(c, st);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "combine launch");
  return timing_end(tl, st);
}

}  // namespace

extern "C" {

int mer_hip_abi_version(void) { return MER_ABI_VERSION; }

int mer_hip_init(int device) {
  std::lock_guard<std::mutex> lock(g_mu);
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(MER_ERR_DEVICE_LOST, "no HIP device available");
  if (device < 0 || device >= n || device >= 64) return fail(MER_ERR_WRONG_DEVICE, "device %d out of range (%d devices)", device, n);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_DEVICE_LOST, "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MER_ERR_WRONG_DEVICE, "device %d is %s; this library is built for gfx950 (MI355X) only", device,
                prop.gcnArchName);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_DEVICE_LOST, "hipSetDevice");
  g_dev[device].cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  if (const char *w = getenv("MER_WAVES_PER_CU")) {
    const long v = strtol(w, nullptr, 10);
    if (v >= 1 && v <= 64) g_dev[device].waves_per_cu = (uint32_t)v;
  }
  g_dev[device].ready = true;
  g_device = device;
  return ok();
}

int mer_hip_shutdown(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_device < 0) return MER_OK;
  DeviceState &d = g_dev[g_device];
  (void)hipDeviceSynchronize();
  if (d.scratch) (void)hipFree(d.scratch);
  d = DeviceState{};
  g_device = -1;
  return MER_OK;
}

const char *mer_last_error(void) { return t_err.c_str(); }

int mer_last_error_info(mer_error_info *out) {
  if (out) *out = t_info;
  return t_info.status;
}

int mer_hip_take_device_status(void) {
  int rc = require_init();
  if (rc) return rc;
  uint32_t s = 0;
  hipError_t e = read_and_clear_device_status(&s);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_DEVICE_LOST, "device status readback");
  if (s) return fail((int)s, "a kernel recorded device status %u (residency miss: expert id out of table or not resident)", s);
  return MER_OK;
}

int mer_hip_stage_timing_enable(int enable) {
  int rc = require_init();
  if (rc) return rc;
  g_timing = enable != 0;
  g_timed_used = 0;
  return MER_OK;
}

int mer_hip_stage_timing_read(double *ms, uint64_t *counts) {
  int rc = require_init();
  if (rc) return rc;
  for (int i = 0; i < STAGE_COUNT; ++i) {
    if (ms) ms[i] = 0.0;
    if (counts) counts[i] = 0;
  }
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(e, MER_ERR_DEVICE_LOST, "synchronise for stage timings");
  for (size_t i = 0; i < g_timed_used; ++i) {
    float t = 0.f;
    e = hipEventElapsedTime(&t, g_timed[i].start, g_timed[i].end);
    if (e != hipSuccess) return hip_fail(e, MER_ERR_RUNTIME_INVARIANT, "stage timing elapsed");
    if (ms) ms[g_timed[i].stage] += t;
    if (counts) counts[g_timed[i].stage] += 1;
  }
  g_timed_used = 0;
  return MER_OK;
}

size_t mer_expert_weight_bytes(int dtype, size_t d_model, size_t d_ff) {
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0) return 0;
  return sat_mul(sat_mul(div_ceil(sat_mul(d_model, d_ff), 32), 3), block_bytes(dtype));
}

int mer_validate_expert(int dtype, size_t len, size_t x_len, size_t y_len, size_t d_model, size_t d_ff,
                        size_t tolerance) {
  return validate(dtype, len, x_len, y_len, d_model, d_ff, tolerance);
}

int mer_routed_expert_gpu_compatibility(int dtype, size_t d_model, size_t d_ff) {
  if (d_model > MER_MAX_EXPERT_DIM || d_ff > MER_MAX_EXPERT_DIM)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "expert shape d_model=%zu d_ff=%zu exceeds %d", d_model, d_ff,
                MER_MAX_EXPERT_DIM);
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  return MER_OK;
}

int mer_hip_dequantize(int dtype, const void *d_src, size_t src_len, size_t n_weights, float *d_dst, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  const size_t need = sat_mul(div_ceil(n_weights, 32), block_bytes(dtype));
  if (src_len < need) return fail_size(MER_ERR_BUFFER_TOO_SMALL, src_len, need, 0, 0);
  if (n_weights && (!d_src || !d_dst)) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  hipError_t e = launch_dequant(fmt_of(dtype), (const uint8_t *)d_src, n_weights, d_dst, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "dequantize launch");
  return MER_OK;
}

int mer_hip_q4_0_matvec(const void *d_weights, size_t weights_len, size_t w_block_off, size_t rows, size_t columns,
                        const float *d_input, float *d_output, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  // validate_raw_case (q4_parity.rs:621-653)
  if (rows == 0 || columns == 0) return fail(MER_ERR_INVALID_LAYOUT, "Q4_0 raw dispatch requires non-zero rows and columns");
  if (columns % 32) return fail(MER_ERR_INVALID_LAYOUT, "Q4_0 raw dispatch columns %zu are not a multiple of 32", columns);
  const size_t bpr = columns / 32;
  size_t accessed, required;
  if (!checked_mul(rows, bpr, &accessed) || accessed > SIZE_MAX - w_block_off ||
      !checked_mul(accessed + w_block_off, 18, &required))
    return fail(MER_ERR_INVALID_LAYOUT, "Q4_0 raw geometry overflow");
  if (weights_len < required || weights_len % 18)
    return fail(MER_ERR_INVALID_LAYOUT, "Q4_0 raw weights have %zu bytes, require at least %zu complete 18-byte blocks",
                weights_len, required);
  if (rows > UINT32_MAX || bpr > UINT32_MAX) return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "raw matvec too large");
  hipError_t e = launch_q4_raw((const uint8_t *)d_weights, w_block_off, (uint32_t)rows, (uint32_t)bpr, d_input,
                               d_output, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "raw matvec launch");
  return MER_OK;
}

int mer_hip_expert_forward(int dtype, const void *d_bytes, size_t len, const float *d_x, size_t x_len,
                           size_t d_model, size_t d_ff, float *d_y, size_t y_len, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  rc = validate(dtype, len, x_len, y_len, d_model, d_ff, 0);
  if (rc) return rc;
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (d_model == 0) return MER_OK;
  if (d_ff == 0) {
    hipError_t e = hipMemsetAsync(d_y, 0, d_model * sizeof(float), st);
    return e == hipSuccess ? MER_OK : hip_fail(e, MER_ERR_SUBMISSION, "zero output");
  }
  if (!d_bytes || !d_x || !d_y) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  return run_experts(dtype, d_model, d_ff, 1, 1, nullptr, 0, nullptr, (const uint8_t *)d_bytes, nullptr, d_x, d_y,
                     0u, st, true);
}

int mer_hip_expert_forward_host(int dtype, const void *bytes, size_t len, const float *x, size_t x_len,
                                size_t d_model, size_t d_ff, float *y, size_t y_len) {
  int rc = require_init();
  if (rc) return rc;
  rc = validate(dtype, len, x_len, y_len, d_model, d_ff, 0);
  if (rc) return rc;
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  if (d_model == 0) return MER_OK;
  if (d_ff == 0) {
    memset(y, 0, d_model * sizeof(float));
    return MER_OK;
  }
  const size_t need = mer_expert_weight_bytes(dtype, d_model, d_ff);
  void *db = nullptr;
  float *dx = nullptr, *dy = nullptr;
  hipError_t e = hipMalloc(&db, need);
  if (e == hipSuccess) e = hipMalloc(&dx, d_model * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&dy, d_model * sizeof(float));
  if (e != hipSuccess) {
    (void)hipFree(db);
    (void)hipFree(dx);
    return hip_fail(e, MER_ERR_PHYSICAL_CAPACITY, "device staging allocation");
  }
  rc = MER_OK;
  e = hipMemcpy(db, bytes, need, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dx, x, d_model * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) rc = hip_fail(e, MER_ERR_UPLOAD, "host-to-device copy");
  if (!rc) rc = run_experts(dtype, d_model, d_ff, 1, 1, nullptr, 0, nullptr, (const uint8_t *)db, nullptr, dx, dy,
                            0u, nullptr, true);
  if (!rc) {
    e = hipMemcpy(y, dy, d_model * sizeof(float), hipMemcpyDeviceToHost);
    if (e != hipSuccess) rc = hip_fail(e, MER_ERR_READBACK_MAP, "device-to-host copy");
  }
  (void)hipFree(db);
  (void)hipFree(dx);
  (void)hipFree(dy);
  return rc;
}

int mer_hip_moe_forward(int dtype, size_t d_model, size_t d_ff, size_t n_tokens, size_t top_k,
                        const void *const *d_expert_table, size_t table_len, const int32_t *d_expert_ids,
                        const float *d_weights, const float *d_x, float *d_out, unsigned flags, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  if (d_model == 0 || d_ff == 0) return fail(MER_ERR_INVALID_LAYOUT, "expert dimensions must be non-zero");
  if (flags & ~3u) return fail(MER_ERR_INVALID_LAYOUT, "unknown flags 0x%x", flags);
  if ((flags & 3u) == 3u) return fail(MER_ERR_INVALID_LAYOUT, "RESIDUAL and ACCUMULATE are exclusive");
  if (n_tokens == 0 || top_k == 0) return MER_OK;
  if (n_tokens * top_k > (1u << 24) || table_len > UINT32_MAX)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "too many expert instances");
  if (!d_expert_table || !d_expert_ids || !d_weights || !d_x || !d_out)
    return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  return run_experts(dtype, d_model, d_ff, (uint32_t)n_tokens, (uint32_t)top_k, d_expert_table, (uint32_t)table_len,
                     d_expert_ids, nullptr, d_weights, d_x, d_out, flags, (hipStream_t)stream, false);
}

int mer_hip_fill_synthetic(int dtype, uint64_t seed, uint64_t expert_index, uint64_t block_begin, uint64_t n_blocks,
                           float scale_lo, float scale_hi, void *d_dst, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  if (((uintptr_t)d_dst & 1u) != 0) return fail(MER_ERR_MISALIGNED, "fill destination must be 2-byte aligned");
  hipError_t e = launch_fill(fmt_of(dtype), seed, expert_index, block_begin, n_blocks, scale_lo, scale_hi,
                             (uint8_t *)d_dst, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "fill launch");
  return MER_OK;
}

}  // extern "C"
