// mer_abi.hip -- extern "C" boundary of the routed-expert SwiGLU FFN
// (declared in include/mer_hip.h).  Host-side validation mirrors the
// reference's typed errors; device work is enqueued on the caller's stream.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
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

// Per-stream workspace.  Everything a device entry point writes besides
// its outputs (scratch, decode counters, release flags, staging) belongs to
// the workspace of the caller's stream, so calls on different streams never
// share device state and may run concurrently, from any host threads.  The
// workspace's mutex is held for the whole host part of a call (validation
// aside), so calls on one stream from several threads are serialised on the
// host and ordered on the device by the stream.
struct Workspace {
  std::mutex mu;
  bool released = false;         // set (under mu) by mer_hip_stream_release / mer_hip_shutdown
  hipStream_t stream = nullptr;
  float *scratch = nullptr;      // h vectors, digit lines, partial sums
  size_t scratch_floats = 0;
  float *stage = nullptr;        // f32 x and y of the f16-view entry point
  size_t stage_floats = 0;
  float *router_buf = nullptr;   // router logits when the caller asks for none
  size_t router_floats = 0;
  uint32_t *counters = nullptr;  // decode counters (zero between launches) + control lines
  size_t counter_words = 0;
  uint64_t *release = nullptr;   // decode release flags (epoch-valued, zero at allocation)
  size_t release_words = 0;
};

// Control lines (kCtlLines, mer_internal.hpp) sit at the end of a
// workspace's counter allocation.

struct DeviceState {
  bool ready = false;
  int cus = 256;
  uint32_t *status = nullptr;
  uint64_t clock_khz = 100000;
  std::atomic<int> occupancy[2][2][2][3][3] = {};  // resident decode workgroups per CU, by (Q8 act, pair, fmt, GG, GD)
  // Device-wide order of persistent decode launches (guarded by
  // g_launch_mu).  The decode grid fills the device and hands items out by
  // static stride, so it needs all of its workgroups resident; two such
  // grids in flight at once could each hold part of the device while
  // waiting for the rest.  Every launch therefore waits (on the GPU) for the
  // previous one, from whichever stream it came: `decode_done` is recorded
  // after each launch on its stream, and a launch on another stream waits
  // for it first.  Grids of one device never overlap, which also orders the
  // calls that share the no-alloc scratch array.  All launches are plain.
  hipEvent_t decode_done = nullptr;
  hipStream_t decode_last = nullptr;
  bool decode_any = false;
  // This device's copy of the no-alloc scratch array (below), from
  // hipGetSymbolAddress at mer_hip_init.
  uint8_t *noalloc_scratch = nullptr;
  // Workspaces are shared: a call holds its stream's workspace for its whole
  // host part, so a concurrent mer_hip_stream_release cannot free the object
  // under it (the call then finds it marked released and fails cleanly).
  std::unordered_map<hipStream_t, std::shared_ptr<Workspace>> ws;  // guarded by g_mu
};
// Lock order: g_mu, then a workspace's mutex.  Code holding a workspace's
// mutex takes only the leaf locks (g_timing_mu, g_trace_mu, g_launch_mu),
// never g_mu.
std::mutex g_mu;
std::atomic<int> g_device{-1};
DeviceState g_dev[64];
// First epochs of new counter allocations (below 2^63; the kernels hand out
// epochs with bit 63 set), so no two workspaces ever share an epoch.
std::atomic<uint64_t> g_host_epoch{0};

// The GPT-OSS SwiGLU gate clamp (set_swiglu_limit, inference.rs:90-99):
// +inf when none is installed; read by every launch that applies SiLU.
std::atomic<float> g_swiglu_limit{__builtin_inff()};

// Serialises the enqueueing of decode launches (a leaf lock).
std::mutex g_launch_mu;

// Decode item trace (tracing aid), a leaf lock.
std::mutex g_trace_mu;
uint64_t *g_trace = nullptr;
uint64_t g_trace_cap = 0;

// GPU stage timings (stage_timing.rs:6-29 analogue): when enabled, every
// gate/up, down and combine launch is bracketed by a pair of events on the
// launch stream; mer_hip_stage_timing_read sums their elapsed times.
enum Stage { STAGE_GATE_UP = 0, STAGE_DOWN = 1, STAGE_COMBINE = 2, STAGE_PREP = 3, STAGE_DECODE = 4, STAGE_COUNT = 5 };
struct TimedLaunch {
  hipEvent_t start, end;
  int stage;
};
std::mutex g_timing_mu;  // leaf lock: guards g_timed / g_timed_used
std::atomic<bool> g_timing{false};
std::vector<TimedLaunch> g_timed;
size_t g_timed_used = 0;

int timing_begin(int stage, hipStream_t st, size_t *slot) {
  *slot = SIZE_MAX;
  if (!g_timing.load()) return MER_OK;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (g_timed_used == g_timed.size()) {
    TimedLaunch t{};
    if (hipEventCreate(&t.start) != hipSuccess || hipEventCreate(&t.end) != hipSuccess)
      return fail(MER_ERR_RUNTIME_INVARIANT, "stage timing event creation failed");
    g_timed.push_back(t);
  }
  const size_t i = g_timed_used++;
  g_timed[i].stage = stage;
  hipError_t e = hipEventRecord(g_timed[i].start, st);
  if (e != hipSuccess) return fail(MER_ERR_SUBMISSION, "stage timing record: %s", hipGetErrorString(e));
  *slot = i;
  return MER_OK;
}

int timing_end(size_t slot, hipStream_t st) {
  if (slot == SIZE_MAX) return MER_OK;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (slot >= g_timed_used) return MER_OK;  // timings were read meanwhile
  hipError_t e = hipEventRecord(g_timed[slot].end, st);
  if (e != hipSuccess) return fail(MER_ERR_SUBMISSION, "stage timing record: %s", hipGetErrorString(e));
  return MER_OK;
}

int require_init() {
  if (g_device.load() < 0) return fail(MER_ERR_NOT_INITIALIZED, "mer_hip_init has not been called");
  return MER_OK;
}

int hip_fail(hipError_t e, int status, const char *what) {
  return fail(status, "%s: %s", what, hipGetErrorString(e));
}

// The workspace of `st` on the current device, created on first use.
std::shared_ptr<Workspace> workspace_for(hipStream_t st) {
  std::lock_guard<std::mutex> lock(g_mu);
  const int dv = g_device.load();
  if (dv < 0) return nullptr;
  auto &slot = g_dev[dv].ws[st];
  if (!slot) {
    slot = std::make_shared<Workspace>();
    slot->stream = st;
  }
  return slot;
}

// A call that locked a workspace released meanwhile (its buffers are gone).
int released_error() {
  return fail(MER_ERR_RUNTIME_INVARIANT,
              "the stream's workspace was released (mer_hip_stream_release / mer_hip_shutdown) while this call "
              "waited for it; release must not overlap calls on that stream");
}

void free_workspace(Workspace &w) {
  (void)hipStreamSynchronize(w.stream);
  if (w.scratch) (void)hipFree(w.scratch);
  if (w.stage) (void)hipFree(w.stage);
  if (w.router_buf) (void)hipFree(w.router_buf);
  if (w.counters) (void)hipFree(w.counters);
  if (w.release) (void)hipFree(w.release);
  w.scratch = w.stage = w.router_buf = nullptr;
  w.counters = nullptr;
  w.release = nullptr;
  w.scratch_floats = w.stage_floats = w.router_floats = w.counter_words = w.release_words = 0;
}

bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Grow one of a workspace's buffers to at least `need` elements (at least
// `min_elems`).  The old buffer is freed after the workspace's stream has
// drained (the only stream that uses it).  With `zero`, the new buffer is
// cleared on that stream.
template <class T>
int ensure_buf(Workspace &w, T **buf, size_t *cap, size_t need, size_t min_elems, bool zero, const char *what) {
  if (*cap >= need) return MER_OK;
  if (capturing(w.stream))
    return fail(MER_ERR_PHYSICAL_CAPACITY,
                "%s must grow, which cannot happen under graph capture: run the same call once before capturing", what);
  if (*buf) {
    hipError_t e = hipStreamSynchronize(w.stream);
    if (e != hipSuccess) return hip_fail(e, MER_ERR_DEVICE_LOST, "synchronise before workspace growth");
    (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
  }
  const size_t want = need < min_elems ? min_elems : need;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(buf), want * sizeof(T));
  if (e != hipSuccess) {
    *buf = nullptr;
    return hip_fail(e, MER_ERR_PHYSICAL_CAPACITY, what);
  }
  if (zero) {
    e = hipMemsetAsync(*buf, 0, want * sizeof(T), w.stream);
    if (e != hipSuccess) return hip_fail(e, MER_ERR_PHYSICAL_CAPACITY, what);
  }
  *cap = want;
  return MER_OK;
}

int ensure_scratch(Workspace &w, size_t floats, float **out) {
  int rc = ensure_buf(w, &w.scratch, &w.scratch_floats, floats, size_t(1) << 20, false, "scratch allocation");
  *out = w.scratch;
  return rc;
}

// Decode counters: `words` per launch plus the control lines, all zero
// between launches (the kernel re-zeroes what it used on exit), except the
// epoch word, which is given a first epoch unique in this process.
int ensure_counters(Workspace &w, size_t words, uint32_t **out) {
  words += kCtlLines * kPollStride;
  const bool grow = w.counter_words < words;
  int rc = ensure_buf(w, &w.counters, &w.counter_words, words, size_t(1) << 16, true, "decode counter allocation");
  if (rc) return rc;
  if (grow) {
    const uint64_t first = ++g_host_epoch;
    uint32_t *ctl = w.counters + w.counter_words - kCtlLines * kPollStride;
    hipError_t e = hipMemcpyAsync(ctl + kCtlEpochLine * kPollStride, &first, sizeof first, hipMemcpyHostToDevice, w.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w.stream);
    if (e != hipSuccess) return hip_fail(e, MER_ERR_PHYSICAL_CAPACITY, "decode counter initialisation");
  }
  *out = w.counters;
  return MER_OK;
}

// Release flags: zeroed when (re)allocated, never cleared by kernels (they
// hold launch epochs, which are unique, and are compared for equality).
int ensure_release(Workspace &w, size_t words, uint64_t **out) {
  int rc = ensure_buf(w, &w.release, &w.release_words, words, size_t(1) << 15, true, "decode release-flag allocation");
  *out = w.release;
  return rc;
}

int g_index(int g) { return g == 16 ? 0 : (g == 32 ? 1 : 2); }

// Choose the decomposition of one projection launch.
ProjPlan plan_projection(size_t rows, size_t cols, bool fused, bool aligned) {
  ProjPlan pl{};
  // Fast path: rows of an even number of blocks (4-byte aligned chunks) and
  // whole 32-row tiles; every configuration of the benchmark qualifies.
  pl.fast = aligned && cols % 64 == 0 && rows % 64 == 0 && cols <= MER_MAX_EXPERT_DIM &&
            rows <= MER_MAX_EXPERT_DIM && rows > 0;
  if (!pl.fast) return pl;
  const uint32_t C = (uint32_t)(cols / 64);
  if (C <= 16) { pl.G = 16; pl.CPL = 1; pl.slices = 1; }
  else if (C <= 32) { pl.G = 32; pl.CPL = 1; pl.slices = 1; }
  else if (fused) {
    pl.G = 64;
    pl.CPL = (int)div_ceil(C, 64);
    pl.slices = 1;
    if (pl.CPL > kMaxCpl) pl.fast = false;
  } else { pl.G = 64; pl.CPL = 1; pl.slices = (uint32_t)div_ceil(C, 64); }
  pl.chunks_per_slice = (uint32_t)div_ceil(C, pl.slices);
  pl.tiles = (uint32_t)(rows / kTileRows);
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

// Geometry of one projection for the decode kernel: lane-group width G,
// column slices of at most 64 chunks, chunks per slice.
struct SliceGeom {
  int G;
  uint32_t slices, cps;
};
SliceGeom slice_geom(uint32_t chunks, uint32_t min_slices = 1) {
  SliceGeom g{};
  g.slices = (uint32_t)div_ceil(chunks, 64);
  if (g.slices < min_slices) g.slices = min_slices;
  g.cps = (uint32_t)div_ceil(chunks, g.slices);
  g.G = g.cps <= 16 ? 16 : (g.cps <= 32 ? 32 : 64);
  return g;
}

bool decode_eligible(size_t dm, size_t dff, const uint8_t *single) {
  if (single && ((uintptr_t)single % 4) != 0) return false;
  return dm % 64 == 0 && dff % 64 == 0 && dm > 0 && dff > 0 && dm <= MER_MAX_EXPERT_DIM && dff <= MER_MAX_EXPERT_DIM;
}

// Geometry and scratch sizes of one persistent decode launch: everything
// but the buffers, which a workspace or the no-alloc scratch provides.
struct DecodePlan {
  DecodeParams p;
  int fmt;
  SliceGeom gg, gd;
  bool pair;  // two-wave workgroups: a tile's two gate/up slices add up in LDS
  bool q8act;  // Q4_0 with Candle's Q8_0 activations (MER_MOE_QMM)
  size_t n_xd, n_gp, n_hd, n_pa;  // floats: x digit lines, gate/up slice partials, h digit lines, down partials
  size_t layer_flags, gd_flags;   // 64-bit release flags
  bool gd_fan;
  size_t floats() const { return n_xd + n_gp + n_hd + n_pa; }
};

void plan_decode(DecodePlan &pl, int dtype, size_t dm, size_t dff, uint32_t n_layers, uint32_t n_tok, uint32_t top_k,
                 const LayerArgs *layers, const uint8_t *single, unsigned flags) {
  DeviceState &dev = g_dev[g_device.load()];
  const int fmt = fmt_of(dtype);
  pl.fmt = fmt;
  pl.q8act = fmt == FMT_Q4_0 && (flags & kFlagQ8Act) != 0;
  DecodeParams &p = pl.p;
  p = DecodeParams{};
  p.swiglu_limit = g_swiglu_limit.load();
  for (uint32_t l = 0; l < n_layers; ++l) p.layers[l] = layers[l];
  p.single = single;
  p.n_layers = n_layers;
  p.n_tok = n_tok;
  p.top_k = top_k;
  p.n_inst = n_tok * top_k;
  p.d_model = (uint32_t)dm;
  p.d_ff = (uint32_t)dff;
  p.flags = flags;
  p.proj_bytes = div_ceil(dm * dff, 32) * block_bytes(dtype);
  p.xblocks = (uint32_t)(dm / 32);
  p.hblocks = (uint32_t)(dff / 32);
  // Narrow layers (fewer than 512 gate/up items, e.g. 8 Qwen3 experts x 24
  // tiles) split gate/up rows into two column slices, so twice as many waves
  // stream each layer's gate and up weights (measured: 1006 -> 1111 tokens/s
  // on the 48-layer Qwen3 decode; wider layers gain nothing).
  const uint32_t g_chunks = (uint32_t)(dm / 64);
  const bool narrow = (uint64_t)n_tok * top_k * (dff / kTileRows) < 512 && g_chunks >= 32;
  pl.gg = slice_geom(g_chunks, narrow ? 2 : 1);
  // Down rows longer than 64 chunks are cut into 32-chunk slices when they
  // divide evenly (Mixtral's 224 -> 7 x 32), so every lane of a 32-lane row
  // group has a chunk, as long as the combine still loads all its parts in
  // one batch (measured on the Mixtral decode: 701 -> 711 tokens/s against
  // 4 slices of 56 chunks).
  const uint32_t d_chunks = (uint32_t)(dff / 64);
  const bool d32 = d_chunks > 64 && d_chunks % 32 == 0 && top_k * (d_chunks / 32) <= kCombineBatch;
  pl.gd = slice_geom(d_chunks, d32 ? d_chunks / 32 : 1);
  p.g_chunks = (uint32_t)(dm / 64);
  p.g_slices = pl.gg.slices;
  p.g_cps = pl.gg.cps;
  p.g_tiles = (uint32_t)(dff / kTileRows);
  p.d_chunks = (uint32_t)(dff / 64);
  p.d_slices = pl.gd.slices;
  p.d_cps = pl.gd.cps;
  p.d_tiles = (uint32_t)(dm / kTileRows);
  const uint32_t pack_blocks = fmt == FMT_Q4_0 ? 16 : 8;
  p.p_items = (uint32_t)div_ceil(p.xblocks, pack_blocks);
  p.combine_packs = 1u;
  p.off_p = n_tok;
  // Gate/up rows cut into two slices of at most 32 chunks run in two-wave
  // workgroups (items 2u and 2u+1 of one unit): the slices of a tile are
  // consecutive items, so with the G items starting at an even index of an
  // even-length layer they always share a workgroup and add up in LDS.
  // Measured: MER_DECODE_NO_PAIR=1 keeps the one-wave layout (A/B).
  static const bool no_pair = [] {
    const char *v = getenv("MER_DECODE_NO_PAIR");
    return v && v[0] == '1';
  }();
  pl.pair = !no_pair && pl.gg.slices == 2 && pl.gg.G <= 32;
  p.off_g = p.off_p + n_tok * p.p_items;
  if (pl.pair && (p.off_g & 1u)) ++p.off_g;  // one padding P item
  p.off_d = p.off_g + p.n_inst * p.g_slices * p.g_tiles;
  p.items_per_layer = p.off_d + p.n_inst * p.d_slices * p.d_tiles;
  if (pl.pair && (p.items_per_layer & 1u)) ++p.items_per_layer;  // one padding D item
  p.total_items = (uint64_t)p.items_per_layer * n_layers;

  // counters per layer.  Polled counters (P[n_tok] G-done[n_inst*d_slices]
  // C-done[n_tok]) sit kPollStride words apart, one per 256-byte line, so waiting
  // waves spread their polls over the memory channels; arrive-only counters
  // (G-arrive[n_inst*g_tiles] D-arrive[n_tok*d_tiles]) are packed after them.
  p.c_p = 0;
  p.c_gd = p.c_p + n_tok * kPollStride;
  p.c_c = p.c_gd + p.n_inst * p.d_slices * kPollStride;
  p.c_ga = p.c_c + n_tok * kPollStride;
  p.c_da = p.c_ga + p.n_inst * p.g_tiles;
  p.cnt_per_layer = (p.c_da + n_tok * p.d_tiles + kPollStride - 1) / kPollStride * kPollStride;
  p.n_counters = p.cnt_per_layer * n_layers;

  auto up64 = [](size_t v) { return (v + 63) / 64 * 64; };
  const size_t L = n_layers;
  pl.n_xd = L * n_tok * p.xblocks * kLineDwords;
  pl.n_gp = p.g_slices > 1 && !pl.pair ? up64(L * p.n_inst * p.g_slices * 2 * dff) : 0;
  pl.n_hd = L * p.n_inst * p.hblocks * kLineDwords;
  pl.n_pa = up64(L * p.n_inst * p.d_slices * dm);
  // Release flags of layers, and of h slices when their count is small
  // (each flag takes a 256-byte line).
  pl.layer_flags = (size_t)n_layers * n_tok * kReleaseFan * kFlagStride;
  const size_t gd_keys = (size_t)n_layers * p.n_inst * p.d_slices;
  pl.gd_fan = gd_keys <= 1024;
  pl.gd_flags = pl.gd_fan ? gd_keys * kReleaseFan * kFlagStride : 0;
  p.status = dev.status;
  p.timeout_ticks = dev.clock_khz * 2000;  // 2 s per wait
  {
    std::lock_guard<std::mutex> lk(g_trace_mu);
    p.trace = g_trace;
    p.trace_cap = g_trace_cap;
  }
}

// Point the plan at its buffers: `f` holds pl.floats() floats, `counters`
// p.n_counters words (zero), `ctl` the three control lines (exit count,
// abort flag, epoch word), `release` the flags.
void bind_decode(DecodePlan &pl, float *f, uint32_t *counters, uint32_t *ctl, uint64_t *release) {
  DecodeParams &p = pl.p;
  p.xq_dig = reinterpret_cast<uint32_t *>(f);
  f += pl.n_xd;
  p.gpart = f;
  f += pl.n_gp;
  p.hq_dig = reinterpret_cast<uint32_t *>(f);
  f += pl.n_hd;
  p.partial = f;
  p.counters = counters;
  p.release = release;
  p.gd_release = pl.gd_fan ? release + pl.layer_flags : nullptr;
  p.exit_count = ctl;
  p.abort_flag = ctl + kPollStride;
  p.exit_groups = ctl + 2 * kPollStride;
  p.epoch_word = reinterpret_cast<uint64_t *>(ctl + kCtlEpochLine * kPollStride);
}

// Grid sizing and the launch itself.
// `prep`, if given, enqueues work on `st` that must run after the previous
// decode launch of the device and before this one (the no-alloc scratch
// preparation).
int launch_planned(DecodePlan &pl, hipStream_t st, const std::function<hipError_t()> &prep = nullptr) {
  DeviceState &dev = g_dev[g_device.load()];
  DecodeParams &p = pl.p;
  const void *fn = decode_kernel_fn(pl.fmt, pl.gg.G, pl.gd.G, pl.pair, pl.q8act);
  const uint32_t wpg = pl.pair ? 2u : 1u;
  std::atomic<int> &occ_slot = dev.occupancy[pl.q8act][pl.pair][pl.fmt][g_index(pl.gg.G)][g_index(pl.gd.G)];
  int occ = occ_slot.load();
  if (occ == 0) {
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, 64 * wpg, 0);
    if (e != hipSuccess || occ <= 0) return hip_fail(e, MER_ERR_RUNTIME_INVARIANT, "decode kernel occupancy query");
    occ_slot.store(occ);
  }
  const uint64_t units = (p.total_items + wpg - 1) / wpg;
  uint64_t grid = (uint64_t)dev.cus * (uint64_t)occ;
  if (grid > units) grid = units;
  if (grid == 0) return MER_OK;
  // unit indices run to units + grid (each workgroup steps once past the end)
  if ((units + grid) * wpg >= (uint64_t)UINT32_MAX)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "decode launch of %llu items exceeds the 32-bit item space",
                (unsigned long long)p.total_items);

  size_t tl = SIZE_MAX;
  hipError_t e;
  {
    std::lock_guard<std::mutex> lk(g_launch_mu);
    // Under graph capture the launch is not ordered here: the caller orders
    // the graph's replays against decode calls on other streams.
    const bool cap = capturing(st);
    if (!cap && dev.decode_any && dev.decode_last != st) {
      e = hipStreamWaitEvent(st, dev.decode_done, 0);
      if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "ordering after the previous decode launch");
    }
    const int trc = timing_begin(STAGE_DECODE, st, &tl);
    if (trc) return trc;
    e = hipSuccess;
    if (prep) e = prep();
    if (e == hipSuccess) e = launch_decode(fn, (uint32_t)grid, wpg, p, st);
    if (e == hipSuccess && !cap) {
      e = hipEventRecord(dev.decode_done, st);
      dev.decode_last = st;
      dev.decode_any = true;
    }
  }
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "decode launch");
  return timing_end(tl, st);
}

// One persistent launch for n_layers MoE layers (fast path) on the
// workspace of the caller's stream.
int run_decode(Workspace &w, int dtype, size_t dm, size_t dff, uint32_t n_layers, uint32_t n_tok, uint32_t top_k,
               const LayerArgs *layers, const uint8_t *single, unsigned flags) {
  DecodePlan pl;
  plan_decode(pl, dtype, dm, dff, n_layers, n_tok, top_k, layers, single, flags);
  float *f = nullptr;
  int rc = ensure_scratch(w, pl.floats(), &f);
  if (rc) return rc;
  uint32_t *counters = nullptr;
  if ((rc = ensure_counters(w, pl.p.n_counters, &counters))) return rc;
  uint64_t *release = nullptr;
  if ((rc = ensure_release(w, pl.layer_flags + pl.gd_flags, &release))) return rc;
  bind_decode(pl, f, counters, counters + w.counter_words - kCtlLines * kPollStride, release);
  return launch_planned(pl, w.stream);
}

// ---- no-allocation decode (mer_hip_moe_forward_noalloc) --------------------
// The decode kernel's scratch for callers that cannot allocate: one array
// per device, held until the process ends.  In host code `scratch` names a
// host-side stand-in; the device address comes from hipGetSymbolAddress
// (DeviceState::noalloc_scratch), which is what kernels and copies use.
// Layout: the kCtlLines control lines (exit count, abort flag, exit-group
// counters, epoch word: a 256-byte line each, at fixed offsets so the epoch
// word survives calls of any shape), then the counters, the release flags
// and the float region of the call.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

int run_decode_noalloc(int dtype, size_t dm, size_t dff, uint32_t n_tok, uint32_t top_k, const LayerArgs &la,
                       unsigned flags, hipStream_t st) {
  DeviceState &dev = g_dev[g_device.load()];
  uint8_t *base = dev.noalloc_scratch;
  if (!base) return fail(MER_ERR_NOT_INITIALIZED, "the no-alloc scratch of this device is not set up");
  DecodePlan pl;
  plan_decode(pl, dtype, dm, dff, 1, n_tok, top_k, &la, nullptr, flags);
  auto up256 = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t ctl_bytes = kCtlLines * kPollStride * 4;
  const size_t cnt_bytes = up256((pl.p.n_counters) * 4);
  const size_t flag_bytes = up256((pl.layer_flags + pl.gd_flags) * 8);
  const size_t float_bytes = up256(pl.floats() * 4);
  const size_t need = ctl_bytes + cnt_bytes + flag_bytes + float_bytes;
  if (need > kNoAllocScratchBytes)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE,
                "the no-alloc decode needs %zu bytes of scratch for d_model=%zu d_ff=%zu n_tokens=%u top_k=%u; its "
                "static scratch holds %zu (use mer_hip_moe_forward, which grows a workspace)",
                need, dm, dff, n_tok, top_k, kNoAllocScratchBytes);
  uint32_t *ctl = reinterpret_cast<uint32_t *>(base);
  uint32_t *counters = reinterpret_cast<uint32_t *>(base + ctl_bytes);
  uint64_t *release = reinterpret_cast<uint64_t *>(base + ctl_bytes + cnt_bytes);
  float *f = reinterpret_cast<float *>(base + ctl_bytes + cnt_bytes + flag_bytes);
  bind_decode(pl, f, counters, ctl, release);
  // The array keeps the last call's contents, laid out for that call's
  // shape: clear the exit count and abort flag, this call's counters and
  // release flags (one kernel, no memset node), and give a never-used epoch
  // word its first epoch.
  return launch_planned(pl, st, [&] {
    return launch_decode_scratch_prep(ctl, kCtlEpochLine * kPollStride, counters, (cnt_bytes + flag_bytes) / 4, pl.p.epoch_word,
                                      st);
  });
}

// Enqueue prep -> gate/up -> down -> combine for n_inst expert instances.
int run_experts(Workspace &w, int dtype, size_t dm, size_t dff, uint32_t n_tokens, uint32_t top_k,
                const void *const *table, uint32_t table_len, const int32_t *ids, const uint8_t *single,
                const float *weights, const float *x, float *out, unsigned flags, bool direct_out) {
  const hipStream_t st = w.stream;
  const int fmt = fmt_of(dtype);
  const uint32_t n_inst = n_tokens * top_k;
  const size_t proj = div_ceil(dm * dff, 32) * block_bytes(dtype);
  const bool aligned = single ? ((uintptr_t)single % 4 == 0) : true;
  if (decode_eligible(dm, dff, single)) {
    LayerArgs la{};
    la.table = table;
    la.table_len = table_len;
    la.ids = ids;
    la.weights = weights;
    la.x = x;
    la.out = out;
    return run_decode(w, dtype, dm, dff, 1, n_tokens, top_k, &la, single, flags);
  }

  const ProjPlan pg = plan_projection(dff, dm, true, aligned);
  const ProjPlan pd = plan_projection(dm, dff, false, aligned);
  const bool fast = pg.fast && pd.fast;
  const uint32_t slices = fast ? pd.slices : 1;
  const bool write_direct = direct_out && slices == 1 && n_inst == 1 && flags == 0;

  // scratch (floats; every region 256-byte aligned):
  //   inst_ptr | x digits + scales | h digits + scales (fast) or f32 h | partials
  auto up64 = [](size_t v) { return (v + 63) / 64 * 64; };
  const size_t xblocks = dm / 32, hblocks = dff / 32;
  const size_t n_ptr = up64(2 * (size_t)n_inst);
  const size_t n_xd = fast ? up64((size_t)n_tokens * xblocks * kBlockDigitDwords) : 0;
  const size_t n_xs = fast ? up64((size_t)n_tokens * xblocks) : 0;
  const size_t n_hd = fast ? up64((size_t)n_inst * hblocks * kBlockDigitDwords) : 0;
  const size_t n_hs = fast ? up64((size_t)n_inst * hblocks) : 0;
  const size_t n_h = fast ? 0 : up64((size_t)n_inst * dff);
  const size_t n_p = write_direct ? 0 : up64((size_t)n_inst * slices * dm);
  float *scr = nullptr;
  int rc = ensure_scratch(w, n_ptr + n_xd + n_xs + n_hd + n_hs + n_h + n_p, &scr);
  if (rc) return rc;
  float *cur = scr;
  const uint8_t **inst_ptr = reinterpret_cast<const uint8_t **>(cur);
  cur += n_ptr;
  uint32_t *xq_dig = reinterpret_cast<uint32_t *>(cur);
  cur += n_xd;
  float *xq_scale = cur;
  cur += n_xs;
  uint32_t *hq_dig = reinterpret_cast<uint32_t *>(cur);
  cur += n_hd;
  float *hq_scale = cur;
  cur += n_hs;
  float *h = cur;
  cur += n_h;
  float *partial = write_direct ? out : cur;

  hipError_t e;
  size_t tl = SIZE_MAX;
  int trc;

  PrepParams q{};
  q.table = table;
  q.table_len = table_len;
  q.ids = ids;
  q.weights = weights;
  q.single = single;
  q.top_k = top_k;
  q.inst_ptr = inst_ptr;
  q.x = x;
  q.d_model = (uint32_t)dm;
  q.blocks = (uint32_t)xblocks;
  q.xq_dig = fast ? xq_dig : nullptr;
  q.xq_scale = xq_scale;
  if ((trc = timing_begin(STAGE_PREP, st, &tl))) return trc;
  e = launch_prep(fmt, q, n_tokens, st);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "prep launch");
  if ((trc = timing_end(tl, st))) return trc;

  // gate/up + SiLU -> h (digit planes on the fast path)
  if ((trc = timing_begin(STAGE_GATE_UP, st, &tl))) return trc;
  if (fast) {
    ProjParams p{};
    p.swiglu_limit = g_swiglu_limit.load();
    p.inst_ptr = inst_ptr;
    p.n_inst = n_inst;
    p.proj_off0 = 0;
    p.proj_off1 = proj;
    p.rows = (uint32_t)dff;
    p.chunks = (uint32_t)(dm / 64);
    p.slices = 1;
    p.chunks_per_slice = pg.chunks_per_slice;
    p.tiles = pg.tiles;
    p.xq_dig = xq_dig;
    p.xq_scale = xq_scale;
    p.xq_blocks = (uint32_t)xblocks;
    p.x_div = top_k;
    p.hq_dig = hq_dig;
    p.hq_scale = hq_scale;
    p.hq_blocks = (uint32_t)hblocks;
    p.out = nullptr;
    e = launch_proj(fmt, true, pg, p, st);
  } else {
    GenericParams g{};
    g.swiglu_limit = g_swiglu_limit.load();
    g.inst_ptr = inst_ptr;
    g.n_inst = n_inst;
    g.proj_off0 = 0;
    g.proj_off1 = proj;
    g.rows = (uint32_t)dff;
    g.cols = (uint32_t)dm;
    g.fused = 1;
    g.x = x;
    g.x_div = top_k;
    g.x_stride = dm;
    g.out = h;
    e = launch_generic(fmt, g, st);
  }
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "gate/up launch");
  if ((trc = timing_end(tl, st))) return trc;

  // down -> partial [inst][slice][dm]
  if ((trc = timing_begin(STAGE_DOWN, st, &tl))) return trc;
  if (fast) {
    ProjParams p{};
    p.swiglu_limit = g_swiglu_limit.load();
    p.inst_ptr = inst_ptr;
    p.n_inst = n_inst;
    p.proj_off0 = 2 * proj;
    p.proj_off1 = 0;
    p.rows = (uint32_t)dm;
    p.chunks = (uint32_t)(dff / 64);
    p.slices = pd.slices;
    p.chunks_per_slice = pd.chunks_per_slice;
    p.tiles = pd.tiles;
    p.xq_dig = hq_dig;
    p.xq_scale = hq_scale;
    p.xq_blocks = (uint32_t)hblocks;
    p.x_div = 1;
    p.out = partial;
    e = launch_proj(fmt, false, pd, p, st);
  } else {
    GenericParams g{};
    g.swiglu_limit = g_swiglu_limit.load();
    g.inst_ptr = inst_ptr;
    g.n_inst = n_inst;
    g.proj_off0 = 2 * proj;
    g.proj_off1 = 0;
    g.rows = (uint32_t)dm;
    g.cols = (uint32_t)dff;
    g.fused = 0;
    g.x = h;
    g.x_div = 1;
    g.x_stride = dff;
    g.out = partial;
    e = launch_generic(fmt, g, st);
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

// Grouped multi-token path: group -> gate/up -> down -> combine.
int run_grouped(Workspace &w, int dtype, size_t dm, size_t dff, uint32_t n_tokens, uint32_t top_k,
                const void *const *table, uint32_t table_len, const int32_t *ids, const float *weights,
                const float *x, float *out, unsigned flags) {
  DeviceState &dev = g_dev[g_device.load()];
  const hipStream_t st = w.stream;
  GroupedParams p{};
  p.swiglu_limit = g_swiglu_limit.load();
  p.table = table;
  p.table_len = table_len;
  p.ids = ids;
  p.weights = weights;
  p.x = x;
  p.out = out;
  p.flags = flags;
  p.q8act = dtype == MER_DTYPE_Q4_0 && (flags & MER_MOE_QMM) ? 1u : 0u;
  p.n_tok = n_tokens;
  p.top_k = top_k;
  p.n_pairs = n_tokens * top_k;
  p.d_model = (uint32_t)dm;
  p.d_ff = (uint32_t)dff;
  p.xblocks = (uint32_t)(dm / 32);
  p.hblocks = (uint32_t)(dff / 32);
  p.proj_bytes = div_ceil(dm * dff, 32) * block_bytes(dtype);
  p.status = dev.status;
  // Token tiles hold <= 16 pairs of one expert: at most n_pairs / 16 full
  // tiles plus one partial tile per distinct expert.
  const uint32_t max_tiles = p.n_pairs / 16 + (p.n_pairs < table_len ? p.n_pairs : table_len);

  auto up64 = [](size_t v) { return (v + 63) / 64 * 64; };  // floats; 256-byte aligned regions
  const size_t n_hdr = 64;
  const size_t n_plist = up64(p.n_pairs);
  const size_t n_ok = up64(p.n_pairs);
  const size_t n_tiles = up64((size_t)max_tiles * sizeof(GroupTile) / 4);
  const size_t n_xg = up64((size_t)n_tokens * p.xblocks * 32);  // 4 k-group records of 8 dwords per block
  const size_t n_hg = up64((size_t)p.n_pairs * p.hblocks * 32);
  const size_t n_pa = up64((size_t)p.n_pairs * dm);
  const size_t total = n_hdr + n_plist + n_ok + n_tiles + n_xg + n_hg + n_pa;
  float *cur = nullptr;
  int rc = ensure_scratch(w, total, &cur);
  if (rc) return rc;
  p.n_tiles = reinterpret_cast<uint32_t *>(cur);
  cur += n_hdr;
  p.plist = reinterpret_cast<uint32_t *>(cur);
  cur += n_plist;
  p.pair_ok = reinterpret_cast<uint32_t *>(cur);
  cur += n_ok;
  p.tiles = reinterpret_cast<GroupTile *>(cur);
  cur += n_tiles;
  p.xg = reinterpret_cast<uint32_t *>(cur);
  cur += n_xg;
  p.hg = reinterpret_cast<uint32_t *>(cur);
  cur += n_hg;
  p.partial = cur;

  const int fmt = fmt_of(dtype);
  size_t tl = SIZE_MAX;
  int trc;
  hipError_t e;
  if ((trc = timing_begin(STAGE_PREP, st, &tl))) return trc;
  if ((e = launch_grouped_prep(p, st)) != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "grouping launch");
  if ((trc = timing_end(tl, st))) return trc;
  if ((trc = timing_begin(STAGE_GATE_UP, st, &tl))) return trc;
  if ((e = launch_grouped_proj(fmt, true, p, max_tiles, st)) != hipSuccess)
    return hip_fail(e, MER_ERR_SUBMISSION, "grouped gate/up launch");
  if ((trc = timing_end(tl, st))) return trc;
  if ((trc = timing_begin(STAGE_DOWN, st, &tl))) return trc;
  if ((e = launch_grouped_proj(fmt, false, p, max_tiles, st)) != hipSuccess)
    return hip_fail(e, MER_ERR_SUBMISSION, "grouped down launch");
  if ((trc = timing_end(tl, st))) return trc;
  if ((trc = timing_begin(STAGE_COMBINE, st, &tl))) return trc;
  if ((e = launch_grouped_combine(p, st)) != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "grouped combine launch");
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
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) == hipSuccess && khz > 0)
    g_dev[device].clock_khz = (uint64_t)khz;
  g_dev[device].status = device_status_ptr();
  if (!g_dev[device].status) return fail(MER_ERR_RUNTIME_INVARIANT, "device status symbol not found");
  if (!g_dev[device].noalloc_scratch) {  // once per device, with the device current
    uint8_t *ptr = nullptr;
    e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e, MER_ERR_RUNTIME_INVARIANT, "no-alloc scratch symbol address");
    g_dev[device].noalloc_scratch = ptr;
  }
  if (!g_dev[device].decode_done) {
    e = hipEventCreateWithFlags(&g_dev[device].decode_done, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, MER_ERR_RUNTIME_INVARIANT, "decode ordering event");
  }
  g_dev[device].ready = true;
  g_device = device;
  return ok();
}

int mer_hip_shutdown(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  const int dv = g_device.load();
  if (dv < 0) return MER_OK;
  DeviceState &d = g_dev[dv];
  (void)hipDeviceSynchronize();
  for (auto &kv : d.ws) {
    std::lock_guard<std::mutex> wl(kv.second->mu);
    free_workspace(*kv.second);
    kv.second->released = true;
  }
  d.ws.clear();
  d.ready = false;
  g_device = -1;
  return MER_OK;
}

int mer_hip_stream_release(void *stream) {
  int rc = require_init();
  if (rc) return rc;
  std::shared_ptr<Workspace> w;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto &map = g_dev[g_device.load()].ws;
    auto it = map.find((hipStream_t)stream);
    if (it == map.end()) return MER_OK;
    w = std::move(it->second);
    map.erase(it);
  }
  std::lock_guard<std::mutex> wl(w->mu);  // waits for a call still enqueueing on it
  free_workspace(*w);
  w->released = true;
  return MER_OK;
}

int mer_set_swiglu_limit(float limit) {
  // set_swiglu_limit (inference.rs:90-99): a positive finite limit installs
  // the clamp; anything else removes it.
  g_swiglu_limit.store((limit > 0.0f && limit < __builtin_inff()) ? limit : __builtin_inff());
  return MER_OK;
}

float mer_get_swiglu_limit(void) { return g_swiglu_limit.load(); }

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
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timing = enable != 0;
  g_timed_used = 0;
  return MER_OK;
}

int mer_hip_decode_trace(void *d_records, size_t capacity, uint64_t *clock_khz) {
  int rc = require_init();
  if (rc) return rc;
  {
    std::lock_guard<std::mutex> lk(g_trace_mu);
    g_trace = reinterpret_cast<uint64_t *>(d_records);
    g_trace_cap = d_records ? capacity : 0;
  }
  if (clock_khz) *clock_khz = g_dev[g_device.load()].clock_khz;
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
  std::lock_guard<std::mutex> lk(g_timing_mu);
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

int mer_output_digest(uint64_t token_idx, uint32_t expert_id, const float *y, size_t n, uint64_t *digest,
                      float *out_norm) {
  // summarise_output (inference.rs:3087-3106): FNV-1a-style fold over the
  // f32 bit patterns seeded with the token and expert, and the f64 L2 norm.
  if (n && !y) return fail(MER_ERR_INVALID_LAYOUT, "null output vector");
  double sum_sq = 0.0;
  uint64_t d = 0xcbf29ce484222325ull ^ token_idx ^ (uint64_t)expert_id;
  for (size_t i = 0; i < n; ++i) {
    uint32_t bits;
    memcpy(&bits, &y[i], 4);
    sum_sq += (double)y[i] * (double)y[i];
    d = (d ^ (uint64_t)bits) * 0x100000001b3ull;
  }
  if (digest) *digest = d;
  if (out_norm) *out_norm = (float)__builtin_sqrt(sum_sq);
  return MER_OK;
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
  if (!d_weights || !d_input || !d_output) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
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
  if (d_ff == 0) {  // y = W_down * h over an empty h: zeros (a kernel, so the call can be graph-captured)
    if (!d_y) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
    hipError_t e = launch_zero(d_y, d_model, st);
    return e == hipSuccess ? MER_OK : hip_fail(e, MER_ERR_SUBMISSION, "zero output");
  }
  if (!d_bytes || !d_x || !d_y) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  std::shared_ptr<Workspace> w = workspace_for(st);
  if (!w) return require_init();
  std::lock_guard<std::mutex> wl(w->mu);
  if (w->released) return released_error();
  return run_experts(*w, dtype, d_model, d_ff, 1, 1, nullptr, 0, nullptr, (const uint8_t *)d_bytes, nullptr, d_x, d_y,
                     0u, true);
}

// MER_MOE_QMM runs on the persistent decode kernel and the grouped path
// (both need multiples of 64).  It changes Q4_0 experts alone: the engine's
// use_qmm switches only the Q4_0 arm of dispatch_expert_forward
// (engine.rs:1825-1830), so Q8_0 ignores it.
static int check_qmm(int dtype, size_t d_model, size_t d_ff, unsigned flags) {
  if (!(flags & MER_MOE_QMM) || dtype != MER_DTYPE_Q4_0) return MER_OK;
  if (d_model % 32 || d_ff % 32)
    return fail(MER_ERR_INVALID_LAYOUT,
                "Q4_0 QMatMul requires d_model and d_ff to be multiples of 32, got d_model=%zu, d_ff=%zu", d_model, d_ff);
  if (!decode_eligible(d_model, d_ff, nullptr))
    return fail(MER_ERR_INVALID_LAYOUT,
                "the GPU QMatMul path runs on the decode kernel: d_model and d_ff must be multiples of 64, got %zu, %zu",
                d_model, d_ff);
  return MER_OK;
}

int mer_hip_expert_forward_qmm(const void *d_bytes, size_t len, const float *d_x, size_t x_len, size_t d_model,
                               size_t d_ff, float *d_y, size_t y_len, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  rc = validate(MER_DTYPE_Q4_0, len, x_len, y_len, d_model, d_ff, 0);
  if (rc) return rc;
  if (d_model == 0 || d_ff == 0) return fail(MER_ERR_INVALID_LAYOUT, "expert dimensions must be non-zero");
  if ((rc = check_qmm(MER_DTYPE_Q4_0, d_model, d_ff, MER_MOE_QMM))) return rc;
  if (!d_bytes || !d_x || !d_y) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  if ((uintptr_t)d_bytes % 4)
    return fail(MER_ERR_MISALIGNED, "the GPU QMatMul path needs 4-byte aligned expert bytes");
  hipStream_t st = (hipStream_t)stream;
  std::shared_ptr<Workspace> w = workspace_for(st);
  if (!w) return require_init();
  std::lock_guard<std::mutex> wl(w->mu);
  if (w->released) return released_error();
  return run_experts(*w, MER_DTYPE_Q4_0, d_model, d_ff, 1, 1, nullptr, 0, nullptr, (const uint8_t *)d_bytes, nullptr,
                     d_x, d_y, MER_MOE_QMM, true);
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
  if (!rc) {
    std::shared_ptr<Workspace> w = workspace_for(nullptr);
    if (!w) {
      rc = require_init();
    } else {
      std::lock_guard<std::mutex> wl(w->mu);
      rc = w->released ? released_error() : run_experts(*w, dtype, d_model, d_ff, 1, 1, nullptr, 0, nullptr, (const uint8_t *)db, nullptr, dx, dy, 0u,
                       true);
    }
  }
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
  if (flags & ~(3u | MER_MOE_QMM))
    return fail(MER_ERR_INVALID_LAYOUT, "unknown flags 0x%x (CHAIN applies to mer_hip_moe_forward_layers)", flags);
  if ((flags & 3u) == 3u) return fail(MER_ERR_INVALID_LAYOUT, "RESIDUAL and ACCUMULATE are exclusive");
  if ((rc = check_qmm(dtype, d_model, d_ff, flags))) return rc;
  if (n_tokens == 0 || top_k == 0) return MER_OK;
  if (n_tokens * top_k > (1u << 16) || table_len > UINT32_MAX)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "too many expert instances");
  if (!d_expert_table || !d_expert_ids || !d_weights || !d_x || !d_out)
    return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  std::shared_ptr<Workspace> w = workspace_for((hipStream_t)stream);
  if (!w) return require_init();
  std::lock_guard<std::mutex> wl(w->mu);
  if (w->released) return released_error();
  return run_experts(*w, dtype, d_model, d_ff, (uint32_t)n_tokens, (uint32_t)top_k, d_expert_table,
                     (uint32_t)table_len, d_expert_ids, nullptr, d_weights, d_x, d_out, flags, false);
}

int mer_hip_moe_forward_noalloc(int dtype, size_t d_model, size_t d_ff, size_t n_tokens, size_t top_k,
                                const void *const *d_expert_table, size_t table_len, const int32_t *d_expert_ids,
                                const float *d_weights, const float *d_x, float *d_out, unsigned flags,
                                void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  if (flags & ~(3u | MER_MOE_QMM)) return fail(MER_ERR_INVALID_LAYOUT, "unknown flags 0x%x", flags);
  if ((flags & 3u) == 3u) return fail(MER_ERR_INVALID_LAYOUT, "RESIDUAL and ACCUMULATE are exclusive");
  if (!decode_eligible(d_model, d_ff, nullptr))
    return fail(MER_ERR_INVALID_LAYOUT,
                "the no-alloc entry point runs the decode kernel only: d_model and d_ff must be non-zero multiples "
                "of 64, got %zu, %zu",
                d_model, d_ff);
  if (n_tokens == 0 || top_k == 0) return MER_OK;
  if (n_tokens * top_k > (1u << 16) || table_len > UINT32_MAX)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "too many expert instances");
  if (!d_expert_table || !d_expert_ids || !d_weights || !d_x || !d_out)
    return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  LayerArgs la{};
  la.table = d_expert_table;
  la.table_len = (uint32_t)table_len;
  la.ids = d_expert_ids;
  la.weights = d_weights;
  la.x = d_x;
  la.out = d_out;
  return run_decode_noalloc(dtype, d_model, d_ff, (uint32_t)n_tokens, (uint32_t)top_k, la, flags,
                            (hipStream_t)stream);
}

int mer_hip_expert_batch_f16(int dtype, size_t d_model, size_t d_ff, size_t n_experts,
                             const void *const *d_expert_table, size_t table_len, const int32_t *d_expert_ids,
                             const uint16_t *d_x, uint16_t *d_out, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  if (d_model == 0 || d_ff == 0) return fail(MER_ERR_INVALID_LAYOUT, "expert dimensions must be non-zero");
  if (n_experts == 0) return MER_OK;
  if (n_experts > (1u << 16) || table_len > UINT32_MAX)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "too many experts in one batch");
  if (!d_expert_table || !d_expert_ids || !d_x || !d_out) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  // Each expert is a one-slot token of weight 1 on its own copy of x, so
  // the routed forward's output row i is y of expert i, uncombined.
  const hipStream_t st = (hipStream_t)stream;
  std::shared_ptr<Workspace> w = workspace_for(st);
  if (!w) return require_init();
  std::lock_guard<std::mutex> wl(w->mu);
  if (w->released) return released_error();
  const size_t need = 2 * n_experts * d_model;
  rc = ensure_buf(*w, &w->stage, &w->stage_floats, need, 0, false, "f16 staging allocation");
  if (rc) return rc;
  float *x32 = w->stage, *y32 = w->stage + n_experts * d_model;
  hipError_t e = launch_f16_in(d_x, d_model, n_experts, x32, st);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "f16 input staging launch");
  rc = run_experts(*w, dtype, d_model, d_ff, (uint32_t)n_experts, 1u, d_expert_table, (uint32_t)table_len,
                   d_expert_ids, nullptr, nullptr, x32, y32, 0u, false);
  if (rc) return rc;
  e = launch_f16_out(y32, n_experts * d_model, d_out, st);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "f16 output staging launch");
  return MER_OK;
}

int mer_hip_moe_grouped(int dtype, size_t d_model, size_t d_ff, size_t n_tokens, size_t top_k,
                        const void *const *d_expert_table, size_t table_len, const int32_t *d_expert_ids,
                        const float *d_weights, const float *d_x, float *d_out, unsigned flags, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  if (flags & ~(3u | MER_MOE_QMM)) return fail(MER_ERR_INVALID_LAYOUT, "unknown flags 0x%x", flags);
  if ((flags & 3u) == 3u) return fail(MER_ERR_INVALID_LAYOUT, "RESIDUAL and ACCUMULATE are exclusive");
  if (d_model == 0 || d_ff == 0 || d_model % 64 || d_ff % 64)
    return fail(MER_ERR_INVALID_LAYOUT, "the grouped path needs d_model and d_ff to be non-zero multiples of 64, got %zu, %zu",
                d_model, d_ff);
  if (n_tokens == 0 || top_k == 0) return MER_OK;
  if (n_tokens * top_k > kMaxGroupedPairs)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "the grouped path takes at most %u routed pairs, got %zu",
                kMaxGroupedPairs, n_tokens * top_k);
  if (table_len == 0 || table_len > kMaxGroupedExperts)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "the grouped path takes expert tables of 1..%u entries, got %zu",
                kMaxGroupedExperts, table_len);
  if (!d_expert_table || !d_expert_ids || !d_weights || !d_x || !d_out)
    return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  std::shared_ptr<Workspace> w = workspace_for((hipStream_t)stream);
  if (!w) return require_init();
  std::lock_guard<std::mutex> wl(w->mu);
  if (w->released) return released_error();
  return run_grouped(*w, dtype, d_model, d_ff, (uint32_t)n_tokens, (uint32_t)top_k, d_expert_table,
                     (uint32_t)table_len, d_expert_ids, d_weights, d_x, d_out, flags);
}

int mer_hip_moe_forward_layers(int dtype, size_t d_model, size_t d_ff, size_t n_layers, size_t n_tokens,
                               size_t top_k, const mer_layer_args *layers, unsigned flags, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  rc = mer_routed_expert_gpu_compatibility(dtype, d_model, d_ff);
  if (rc) return rc;
  if ((rc = check_qmm(dtype, d_model, d_ff, flags))) return rc;
  if (flags & ~(MER_MOE_RESIDUAL | MER_MOE_ACCUMULATE | MER_MOE_CHAIN | MER_MOE_ROUTE_AFTER_PREV | MER_MOE_QMM))
    return fail(MER_ERR_INVALID_LAYOUT, "unknown flags 0x%x", flags);
  if ((flags & 3u) == 3u) return fail(MER_ERR_INVALID_LAYOUT, "RESIDUAL and ACCUMULATE are exclusive");
  if (n_layers == 0 || n_tokens == 0 || top_k == 0) return MER_OK;
  if (n_layers > kMaxLayers) return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "at most %u layers per call", kMaxLayers);
  if (!decode_eligible(d_model, d_ff, nullptr))
    return fail(MER_ERR_INVALID_LAYOUT,
                "multi-layer decode needs d_model and d_ff multiples of 64 (single-layer calls accept any shape)");
  if (n_tokens * top_k > (1u << 16) || !layers) return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "too many expert instances");
  LayerArgs la[kMaxLayers];
  for (size_t l = 0; l < n_layers; ++l) {
    const mer_layer_args &a = layers[l];
    if (!a.expert_table || !a.expert_ids || !a.weights || !a.out || (!a.x && (l == 0 || !(flags & MER_MOE_CHAIN))))
      return fail(MER_ERR_INVALID_LAYOUT, "layer %zu: null device pointer", l);
    if (a.table_len > UINT32_MAX) return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "table too large");
    la[l].table = a.expert_table;
    la[l].table_len = (uint32_t)a.table_len;
    la[l].ids = a.expert_ids;
    la[l].weights = a.weights;
    la[l].x = a.x;
    la[l].out = a.out;
  }
  std::shared_ptr<Workspace> w = workspace_for((hipStream_t)stream);
  if (!w) return require_init();
  std::lock_guard<std::mutex> wl(w->mu);
  if (w->released) return released_error();
  return run_decode(*w, dtype, d_model, d_ff, (uint32_t)n_layers, (uint32_t)n_tokens, (uint32_t)top_k, la, nullptr,
                    flags);
}

int mer_hip_route_linear_gate(const float *d_gate, size_t n_experts, size_t d_model, const float *d_x,
                              size_t n_tokens, size_t top_k, const mer_gate_options *options, int32_t *d_ids,
                              float *d_weights, float *d_logits, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (n_tokens == 0) return MER_OK;
  if (!d_gate || !d_x || !d_ids || !d_weights) return fail(MER_ERR_INVALID_LAYOUT, "null router buffer");
  if (n_experts == 0 || n_experts > kMaxRouterExperts)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "router supports 1..%u experts, got %zu", kMaxRouterExperts, n_experts);
  if (top_k == 0 || top_k > n_experts || top_k > kMaxRouterTopK)
    return fail(MER_ERR_INVALID_LAYOUT, "top_k must be in 1..=min(n_experts, %u), got %zu", kMaxRouterTopK, top_k);
  if (d_model == 0 || d_model > MER_MAX_EXPERT_DIM)
    return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "router d_model must be in 1..=%d, got %zu", MER_MAX_EXPERT_DIM, d_model);
  if (n_tokens > (1u << 18)) return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "the router takes at most 262144 tokens per call");
  RouterParams p{};
  p.gate = d_gate;
  p.x = d_x;
  p.ids = d_ids;
  p.weights = d_weights;
  p.logits = d_logits;
  p.n_experts = (uint32_t)n_experts;
  p.d_model = (uint32_t)d_model;
  p.n_tokens = (uint32_t)n_tokens;
  p.top_k = (uint32_t)top_k;
  p.scoring = 0;
  p.normalise = 1;
  p.n_group = 1;
  p.topk_group = 1;
  p.scaling = 1.0f;
  if (options) {
    if (options->scoring != 0 && options->scoring != 1)
      return fail(MER_ERR_INVALID_LAYOUT, "unknown scoring function %d", options->scoring);
    if (options->n_group > kMaxRouterGroups)
      return fail(MER_ERR_SHAPE_EXCEEDS_WORKSPACE, "router supports at most %u groups", kMaxRouterGroups);
    p.scoring = options->scoring;
    p.normalise = options->normalise_topk != 0;
    p.bias = options->correction_bias;
    p.n_group = options->n_group;
    p.topk_group = options->topk_group;
    p.scaling = options->routed_scaling_factor;
  }
  p.logit_buf = d_logits;
  std::shared_ptr<Workspace> w;
  std::unique_lock<std::mutex> wl;
  if (!d_logits) {
    w = workspace_for((hipStream_t)stream);
    if (!w) return require_init();
    wl = std::unique_lock<std::mutex>(w->mu);
    if (w->released) return released_error();
    rc = ensure_buf(*w, &w->router_buf, &w->router_floats, n_tokens * n_experts, 0, false, "router logits allocation");
    if (rc) return rc;
    p.logit_buf = w->router_buf;
  }
  hipError_t e = launch_router(p, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "router launch");
  return MER_OK;
}

int mer_hip_fill_synthetic(int dtype, uint64_t seed, uint64_t expert_index, uint64_t block_begin, uint64_t n_blocks,
                           float scale_lo, float scale_hi, void *d_dst, void *stream) {
  int rc = require_init();
  if (rc) return rc;
  if (dtype != MER_DTYPE_Q4_0 && dtype != MER_DTYPE_Q8_0)
    return fail(MER_ERR_UNSUPPORTED_DTYPE, "unsupported expert dtype %d", dtype);
  if (n_blocks == 0) return MER_OK;
  if (!d_dst) return fail(MER_ERR_INVALID_LAYOUT, "null device pointer");
  if (((uintptr_t)d_dst & 1u) != 0) return fail(MER_ERR_MISALIGNED, "fill destination must be 2-byte aligned");
  hipError_t e = launch_fill(fmt_of(dtype), seed, expert_index, block_begin, n_blocks, scale_lo, scale_hi,
                             (uint8_t *)d_dst, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, MER_ERR_SUBMISSION, "fill launch");
  return MER_OK;
}

}  // extern "C"

namespace mer {

int report_error(int status, const char *msg) { return fail(status, "%s", msg); }
int report_hip_error(hipError_t e, int status, const char *what) { return hip_fail(e, status, what); }
int check_initialised() { return require_init(); }

}  // namespace mer
