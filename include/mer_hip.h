/*
 * mer_hip.h -- C ABI of the MI355X (gfx950) routed-expert SwiGLU FFN.
 *
 * Drop-in for the expert-execution slice of MER
 * (randyap8-wq/Micro-Expert-Router-SSD-Streamed-MoE-MER).  Every entry
 * point names the reference interface it replaces; paths are relative to
 * rust-engine/src/ of the reference.
 *
 * Conventions
 *   - Plain pointers and sizes only; no C++ or torch types cross the ABI.
 *   - Every function returns a mer_status (0 = MER_OK).  A failing call
 *     records thread-local detail, readable with mer_last_error() /
 *     mer_last_error_info().  Nothing aborts or throws across the ABI.
 *   - "d_" pointers are device pointers (hipMalloc'd on the device made
 *     current by mer_hip_init); "stream" is a hipStream_t passed as
 *     void* (NULL = the null stream).  Device entry points are
 *     asynchronous with respect to the host unless stated otherwise.
 *   - Expert blobs use MER's on-disk layout unchanged: gate || up || down,
 *     each projection an independently block-rounded stream of GGUF
 *     blocks (inference.rs:1089-1146); gate/up are [d_ff x d_model] and
 *     down is [d_model x d_ff], row-major.
 *   - Re-entrant.  Each stream has a workspace of its own (scratch,
 *     decode counters and flags, staging), created on the first call that
 *     uses the stream, so calls on different streams never share device
 *     state and may run concurrently from any host threads (the engine's
 *     parallel expert workers, or several concurrent dispatches, each
 *     with its own stream: backend/mod.rs:1346-1432, :2685-2697).  Calls
 *     on one stream from several threads are serialised by the stream's
 *     workspace lock and run in stream order.  Release a stream's
 *     workspace with mer_hip_stream_release before destroying the stream;
 *     a release must not overlap calls on that stream (such a call fails
 *     with MER_ERR_RUNTIME_INVARIANT).
 *   - The persistent decode kernel (mer_hip_moe_forward[_noalloc],
 *     mer_hip_moe_forward_layers, mer_hip_expert_forward for decode shapes)
 *     hands its work items to its workgroups by static stride, so it needs
 *     its whole grid resident to finish.  The library therefore orders all
 *     decode launches of a device one after another on the GPU, whatever
 *     their streams: a launch on another stream than the previous one
 *     waits (hipStreamWaitEvent, no host blocking) for that launch to end.
 *     Two decode grids are never in flight together; other kernels beside
 *     one only delay it.  The library makes no progress guarantee when a
 *     caller runs its own persistent or spin-waiting kernels on the device
 *     at the same time: a decode wait gives up after 2 s with
 *     MER_ERR_RUNTIME_INVARIANT (never a hang).
 *   - Graph capture: every device entry point may be captured into a HIP
 *     graph once a call of the same shape has run on that stream (the
 *     workspace grows only outside capture; growth under capture fails
 *     with MER_ERR_PHYSICAL_CAPACITY).  Replays are correct: the decode
 *     kernel's epoch lives in device memory and each launch hands the
 *     next one a fresh value.  A captured graph holds the workspace's
 *     buffer addresses: a later call of a larger shape on that stream
 *     (which grows the workspace) or mer_hip_stream_release invalidates
 *     graphs captured on it.  Captured decode launches are not ordered
 *     against decode calls on other streams; the caller orders replays.
 */
#ifndef MER_HIP_H
#define MER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MER_ABI_VERSION 1

/* WeightDtype ordinals (inference.rs:138-236); only the GGUF block
 * formats on the hot path are accepted by this library. */
enum mer_dtype {
  MER_DTYPE_Q4_0 = 4,
  MER_DTYPE_Q8_0 = 5,
};

enum mer_status {
  MER_OK = 0,
  /* ExpertWeightsError (inference.rs:1153-1188) */
  MER_ERR_BUFFER_TOO_SMALL = 1,
  MER_ERR_MISALIGNED = 2,
  MER_ERR_COMPUTE = 3, /* the Candle(String) slot: a compute-side failure */
  MER_ERR_INVALID_LAYOUT = 4,
  MER_ERR_TRUNCATED_PAYLOAD = 5,
  /* GpuExpertDispatchErrorKind (backend/mod.rs:349-361) */
  MER_ERR_RESIDENCY_MISS = 16,
  MER_ERR_PHYSICAL_CAPACITY = 17,
  MER_ERR_UPLOAD = 18,
  MER_ERR_VALIDATION_DISPATCH = 19,
  MER_ERR_SUBMISSION = 20,
  MER_ERR_READBACK_CHANNEL = 21,
  MER_ERR_READBACK_MAP = 22,
  MER_ERR_DEVICE_LOST = 23,
  MER_ERR_RUNTIME_INVARIANT = 24,
  /* RoutedExpertGpuIncompatibility (backend/mod.rs:4621-4719) */
  MER_ERR_UNSUPPORTED_DTYPE = 32,
  MER_ERR_SHAPE_EXCEEDS_WORKSPACE = 33,
  /* library state */
  MER_ERR_NOT_INITIALIZED = 48,
  MER_ERR_WRONG_DEVICE = 49,
  MER_ERR_IO = 50, /* a file could not be opened or read (the reference's io::Error) */
};

/* Detail of the calling thread's last failure.  For BufferTooSmall and
 * TruncatedPayload, have/need/d_model/d_ff carry the reference fields
 * (inference.rs:1157-1186). */
typedef struct mer_error_info {
  int32_t status;
  uint64_t have;
  uint64_t need;
  uint64_t d_model;
  uint64_t d_ff;
} mer_error_info;

/* Largest d_model / d_ff a routed expert may have on the GPU
 * (MAX_EXPERT_D_FF, backend/mod.rs:17). */
#define MER_MAX_EXPERT_DIM 16384

/* ---- library ------------------------------------------------------ */
int mer_hip_abi_version(void);
/* Select and initialise a device; fails with MER_ERR_WRONG_DEVICE unless
 * it is a gfx950 (MI355X).  Replaces GpuBackend construction
 * (backend/mod.rs:2202-2260). */
int mer_hip_init(int device);
int mer_hip_shutdown(void);
/* Free the workspace of `stream` (synchronises that stream).  Call it
 * before destroying a stream the library has used; the next call on the
 * stream creates a new workspace.  No reference counterpart (the
 * reference's dispatch workspaces live as long as their backend). */
int mer_hip_stream_release(void *stream);
const char *mer_last_error(void);
int mer_last_error_info(mer_error_info *out);
/* Device fault word written by kernels (bad expert id, null table entry):
 * returns the first status recorded since the last reset and clears it.
 * Synchronises the device. */
int mer_hip_take_device_status(void);

/* GPU stage timings (the StageTimings analogue, stage_timing.rs:6-29):
 * while enabled, each expert launch is bracketed by HIP events on its
 * stream.  read() synchronises the device and returns, per stage
 * {0 = gate/up + SiLU, 1 = down, 2 = combine, 3 = input packing / expert
 * resolution -- the flat-layout fallback's launches -- and 4 = the
 * persistent decode kernel of the fast path}, the summed milliseconds and launch counts since the last
 * enable/read, then resets.  Timing must not be enabled while the caller
 * captures a HIP graph. */
#define MER_STAGE_COUNT 5 /* 4 = the persistent decode kernel (fast path) */
int mer_hip_stage_timing_enable(int enable);
int mer_hip_stage_timing_read(double *ms /*[MER_STAGE_COUNT]*/, uint64_t *counts /*[MER_STAGE_COUNT]*/);

/* Item trace of the persistent decode kernel (tracing aid, no reference
 * counterpart): while set, every launch writes for item i, at record i of
 * d_records (8 x uint64: item << 32 | XCC id << 16 | low 16 bits of HW_ID,
 * start, inputs ready, digits fetched, walk done, arrived, end, combined
 * (the D item that combined a tile: its sum stored and the next layer's
 * input block packed); wall-clock ticks of *clock_khz kHz, 0 = mark not
 * reached).  NULL disables. */
int mer_hip_decode_trace(void *d_records, size_t capacity, uint64_t *clock_khz);

/* The GPT-OSS SwiGLU gate clamp: set_swiglu_limit / swiglu_limit
 * (inference.rs:86-112).  A positive finite limit makes every later expert
 * forward of this process compute silu(clamp(g, -limit, limit)) * u, as
 * clamp_swiglu_gate and the Q8_0 direct path do (inference.rs:118-123,
 * :3689-3702); any other value (0, negative, NaN, inf) removes the clamp,
 * which is the default.  Process-wide, like the reference's global; a call
 * reads it when it enqueues its kernels.  get returns +inf when unset. */
int mer_set_swiglu_limit(float limit);
float mer_get_swiglu_limit(void);

/* ---- host-only sizing and validation (no GPU work) ----------------- */
/* expert_weight_bytes_for (inference.rs:1089-1146); saturates. */
size_t mer_expert_weight_bytes(int dtype, size_t d_model, size_t d_ff);
/* The validation each forward performs before launching:
 *   Q4_0: from_bytes_q4_0_with_tolerance (inference.rs:1766-1783,
 *         :4035-4077) then the x-length check forward_candle performs;
 *   Q8_0: validate_q8_direct_layout (inference.rs:3349-3418). */
int mer_validate_expert(int dtype, size_t len, size_t x_len, size_t y_len,
                        size_t d_model, size_t d_ff, size_t tolerance);
/* summarise_output (inference.rs:3087-3106), the InferenceOutput digest the
 * engine logs per expert output (InferenceOutput, :984-994): digest =
 * FNV-1a-style fold of the f32 bit patterns of y[0..n) seeded with
 * 0xcbf29ce484222325 ^ token_idx ^ expert_id; out_norm = sqrt of the f64
 * sum of squares, rounded to f32.  y is host memory; either output may be
 * NULL. */
int mer_output_digest(uint64_t token_idx, uint32_t expert_id, const float *y, size_t n, uint64_t *digest,
                      float *out_norm);
/* routed_expert_gpu_compatibility (backend/mod.rs:4691-4719), extended:
 * Q8_0 is GPU-eligible here, and any Q4_0 shape is accepted (unaligned
 * shapes run the generic flat-layout kernel). */
int mer_routed_expert_gpu_compatibility(int dtype, size_t d_model, size_t d_ff);

/* ---- device entry points ------------------------------------------ */
/* dequantize_q4_0_to_f32 / dequantize_q8_0_to_f32 (inference.rs:852-868,
 * :963-979): bit-exact d*(q-8) / d*q, tail block truncated. */
int mer_hip_dequantize(int dtype, const void *d_src, size_t src_len,
                       size_t n_weights, float *d_dst, void *stream);

/* Raw Q4_0 qualification matvec (backend/mod.rs:3532-3768,
 * q4_parity.rs:591-619): rows x columns starting at block w_block_off,
 * row r at blocks w_block_off + r*columns/32 ..  */
int mer_hip_q4_0_matvec(const void *d_weights, size_t weights_len,
                        size_t w_block_off, size_t rows, size_t columns,
                        const float *d_input, float *d_output, void *stream);

/* One routed expert, VRAM-resident bytes: drop-in for
 * dispatch_expert_forward's Q4_0 / Q8_0 arms (engine.rs:1761-1848):
 *   Q4_0 -> q4_0_cpu_reference_forward (inference.rs:3291-3306)
 *   Q8_0 -> forward_q8_0_direct_into  (inference.rs:3636-3746)
 * y = W_down (silu(W_gate x) * (W_up x)); fp32 accumulate. */
int mer_hip_expert_forward(int dtype, const void *d_bytes, size_t len,
                           const float *d_x, size_t x_len, size_t d_model,
                           size_t d_ff, float *d_y, size_t y_len, void *stream);

/* dispatch_expert_forward's Q4_0 arm with use_qmm (engine.rs:1825-1830):
 * run_inference_q4_0_qmm / forward_q4_0_qmm_from_exact_bytes
 * (inference.rs:4159-4243) on VRAM-resident Q4_0 bytes, with the arithmetic
 * of MER_MOE_QMM.  Same validation and errors as mer_hip_expert_forward
 * plus MER_ERR_INVALID_LAYOUT for dims that are not multiples of 64 and
 * MER_ERR_MISALIGNED for expert bytes that are not 4-byte aligned (the
 * 22-bit entry point runs those on its flat-layout kernel instead). */
int mer_hip_expert_forward_qmm(const void *d_bytes, size_t len, const float *d_x, size_t x_len, size_t d_model,
                               size_t d_ff, float *d_y, size_t y_len, void *stream);

/* Same with host buffers (copies in, runs, copies out, synchronises):
 * the literal signature of forward_q8_0_direct_into / the Q4_0 reference
 * over ExpertResident::data() bytes.  PCIe-inclusive. */
int mer_hip_expert_forward_host(int dtype, const void *bytes, size_t len,
                                const float *x, size_t x_len, size_t d_model,
                                size_t d_ff, float *y, size_t y_len);

/* Flags for mer_hip_moe_forward. */
#define MER_MOE_RESIDUAL 1u   /* out = x + sum_i w_i y_i                */
#define MER_MOE_ACCUMULATE 2u /* out = out + sum_i w_i y_i              */
/* Q4_0 experts through Candle's QMatMul arithmetic: the engine's default
 * Q4_0 arm (use_qmm_for_q4, engine.rs:1144, :1825-1830 ->
 * run_inference_q4_0_qmm, inference.rs:4159-4243).  Each projection's
 * input (x, then h) is quantised to Q8_0 per 32-element block (candle-core
 * 0.10.2 BlockQ8_0::from_float: d = max|v| / 127 rounded to f16, q =
 * round(v / d) half away from zero) and every block contributes
 * sum_i (w_i - 8) q_i * d_w * d_x, as BlockQ4_0::vec_dot does; the block
 * sums are exact and only their f32 sum order differs from Candle's.
 * Accepted by mer_hip_moe_forward, _noalloc, _layers and _grouped; Q8_0
 * experts ignore it (use_qmm only switches the Q4_0 arm); d_model and d_ff
 * must be multiples of 64 (MER_ERR_INVALID_LAYOUT otherwise; not multiples of 32 is
 * the reference's own InvalidLayout, inference.rs:4211-4215). */
#define MER_MOE_QMM 16u

/* Fused routed experts + top-k weighted combine for n_tokens decode
 * tokens: the WeightedInto loop of moe_step_inner (engine.rs:5548-5639)
 * and routed_expert_matmul_batch_q4 (backend/mod.rs:4401-4418).
 *   d_expert_table[table_len]  device array of device pointers to expert
 *                              blobs (NULL = not resident)
 *   d_expert_ids[n_tokens*top_k], d_weights[n_tokens*top_k]  (device)
 *   d_x[n_tokens*d_model] in, d_out[n_tokens*d_model] out.
 * Combine order per token: acc = 0; acc += w_i * y_i for i in slot order
 * (combine_outputs_into, inference.rs:4472-4491); then the flags.
 * An id >= table_len or a NULL entry contributes nothing and records
 * MER_ERR_RESIDENCY_MISS in the device status word. */
int mer_hip_moe_forward(int dtype, size_t d_model, size_t d_ff,
                        size_t n_tokens, size_t top_k,
                        const void *const *d_expert_table, size_t table_len,
                        const int32_t *d_expert_ids, const float *d_weights,
                        const float *d_x, float *d_out, unsigned flags,
                        void *stream);

/* mer_hip_moe_forward for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No reference counterpart: the reference's dispatch paths own
 * their workspaces.  Same arguments, combine, flags and errors as
 * mer_hip_moe_forward, for shapes the persistent decode kernel runs
 * (d_model and d_ff non-zero multiples of 64).  Its scratch is one static
 * 8 MiB device array per GPU, held until the process ends; a call whose
 * scratch would exceed it fails with MER_ERR_SHAPE_EXCEEDS_WORKSPACE (a
 * Mixtral-shape top-2 token needs 0.41 MiB, so up to 19 such tokens fit).  The call allocates
 * nothing and enqueues two kernels (scratch preparation, decode).  Every
 * call on a GPU shares that GPU's array, which keeps the last call's
 * contents.  Calls from any streams and threads are ordered on the GPU
 * like every decode launch (see the conventions above), so they never
 * overlap; under graph capture that ordering is the caller's: replays of
 * graphs holding no-alloc calls must not overlap other no-alloc calls on
 * the same GPU. */
int mer_hip_moe_forward_noalloc(int dtype, size_t d_model, size_t d_ff,
                                size_t n_tokens, size_t top_k,
                                const void *const *d_expert_table, size_t table_len,
                                const int32_t *d_expert_ids, const float *d_weights,
                                const float *d_x, float *d_out, unsigned flags,
                                void *stream);

/* The GPU backend's f16-view entry points: Backend::expert_matmul /
 * routed_expert_matmul (backend/mod.rs:1095-1103, :4421-4441) for one
 * expert and routed_expert_matmul_batch_q4 (backend/mod.rs:3770-3850,
 * :4401-4418) for a layer batch.  Every expert d_expert_ids[i] (an index
 * into d_expert_table, as for mer_hip_moe_forward) runs on the same f16
 * hidden state d_x [d_model]; d_out [n_experts][d_model] receives each
 * expert's own y, rounded to f16, with no combine.  The reference's batch
 * takes exactly 8 experts and reports any other count as ineligible; this
 * entry point takes any count from 1 (n_experts = 1 is expert_matmul).
 * Errors as mer_hip_moe_forward; a missing expert is recorded in the
 * device status and gives a zero row. */
int mer_hip_expert_batch_f16(int dtype, size_t d_model, size_t d_ff, size_t n_experts,
                             const void *const *d_expert_table, size_t table_len, const int32_t *d_expert_ids,
                             const uint16_t *d_x, uint16_t *d_out, void *stream);

/* Grouped path for multi-token batches (prefill): the same contract as
 * mer_hip_moe_forward -- per token out = [x +] sum_i w_i y_i in slot order,
 * zero-weight slots skipped, misses recorded in the device status -- but
 * the routed (token, slot) pairs are grouped by expert on the device, so
 * every expert's weights are read once for all of its tokens and the
 * projections run as int8 MFMA contractions over token tiles of 16.  This
 * is the batched counterpart of routed_expert_matmul_batch_q4
 * (backend/mod.rs:4401-4418) and of the per-pair dispatch loop of
 * forward_moe_resident_cpu (engine.rs:1761-1848) over a prefill batch.
 * Requires d_model and d_ff to be multiples of 64, n_tokens * top_k <=
 * 4096 and table_len <= 4096.  Inputs are held in 24-bit block fixed
 * point (error <= 2^-24 of each 32-element block's maximum). */
int mer_hip_moe_grouped(int dtype, size_t d_model, size_t d_ff,
                        size_t n_tokens, size_t top_k,
                        const void *const *d_expert_table, size_t table_len,
                        const int32_t *d_expert_ids, const float *d_weights,
                        const float *d_x, float *d_out, unsigned flags,
                        void *stream);

/* Per-layer arguments of mer_hip_moe_forward_layers (device pointers). */
typedef struct mer_layer_args {
  const void *const *expert_table; /* [table_len] expert blob pointers    */
  size_t table_len;
  const int32_t *expert_ids;       /* [n_tokens * top_k]                  */
  const float *weights;            /* [n_tokens * top_k]                  */
  const float *x;                  /* [n_tokens][d_model]; ignored for    */
                                   /* layers > 0 under MER_MOE_CHAIN      */
  float *out;                      /* [n_tokens][d_model]                 */
} mer_layer_args;

#define MER_MOE_CHAIN 4u /* layer l > 0 reads layer l-1's out as its x */
/* Layer l > 0 reads its routing (expert_ids, expert_table) and streams its
 * experts' weights only after layer l-1's output is complete, as a step
 * whose routing is computed from that output must.  Without this flag the
 * launch may start streaming layer l's weights while layer l-1 finishes
 * (the routing of every layer is an input of the launch). */
#define MER_MOE_ROUTE_AFTER_PREV 8u

/* n_layers (<= 64) routed-expert MoE layers of one decode step in a single
 * persistent launch: the per-layer WeightedInto step of moe_step_inner
 * (engine.rs:5548-5639) run for every layer of the model (model.rs:
 * 2715-2741) without returning to the host.  Layers execute in order
 * (layer l starts reading its input only after layer l-1 has written its
 * output), with the same combine order and flags as mer_hip_moe_forward;
 * under MER_MOE_CHAIN layer l's input is layer l-1's out.  Requires
 * d_model and d_ff to be multiples of 64.  The launch sizes its grid to
 * fill every CU; its workgroups take items by static stride, so it runs
 * after any earlier decode launch of the device (see the conventions);
 * ordinary kernels on other streams share the CUs and only slow it. */
int mer_hip_moe_forward_layers(int dtype, size_t d_model, size_t d_ff, size_t n_layers, size_t n_tokens,
                               size_t top_k, const mer_layer_args *layers, unsigned flags, void *stream);

/* ---- routing -------------------------------------------------------- */
/* Options of the LinearGate routing surface (LinearGate::with_routing,
 * gating.rs:207-268).  NULL options = LinearGate::new: softmax scoring,
 * renormalised top-k, no bias, no groups, unit scaling. */
typedef struct mer_gate_options {
  int32_t scoring;              /* 0 = softmax, 1 = sigmoid (ScoringFunc)   */
  int32_t normalise_topk;       /* nonzero: divide the top-k weights by     */
                                /* their sum when it is finite and > 0      */
  const float *correction_bias; /* device [n_experts], added to selection   */
                                /* scores only; NULL = none                 */
  uint32_t n_group;             /* group-limited selection (n_group,        */
  uint32_t topk_group;          /* topk_group); n_group <= 1 disables it    */
  float routed_scaling_factor;  /* applied to the final weights if != 1     */
} mer_gate_options;

#define MER_MAX_ROUTER_EXPERTS 1024
#define MER_MAX_ROUTER_TOP_K 64

/* LinearGate::route_with_scratch (gating.rs:395-476) for n_tokens hidden
 * states on the device: logits = W x, scores, optional bias and group
 * filter, deterministic top-k (higher score first, lower id on ties),
 * weights = unbiased scores renormalised and scaled.
 *   d_gate[n_experts * d_model] (row-major f32), d_x[n_tokens * d_model];
 *   d_ids / d_weights [n_tokens * top_k]: slots beyond the experts with a
 *   finite score get id -1 and weight 0 (the routed forwards skip them);
 *   d_logits [n_tokens * n_experts] or NULL.
 * n_experts <= MER_MAX_ROUTER_EXPERTS, top_k <= MER_MAX_ROUTER_TOP_K,
 * d_model <= MER_MAX_EXPERT_DIM, n_tokens <= 262144.  Without d_logits the
 * library keeps the logits in a buffer of its own (grown on first use, so
 * make one call of the largest shape before capturing a HIP graph). */
int mer_hip_route_linear_gate(const float *d_gate, size_t n_experts, size_t d_model, const float *d_x,
                              size_t n_tokens, size_t top_k, const mer_gate_options *options, int32_t *d_ids,
                              float *d_weights, float *d_logits, void *stream);

/* Synthetic bench / test data: fill n_blocks GGUF blocks of expert
 * `expert_index` starting at block `block_begin` with this library's
 * counter-based generator (nibbles / int8 uniform, d = f16(U(lo,hi))). */
int mer_hip_fill_synthetic(int dtype, uint64_t seed, uint64_t expert_index,
                           uint64_t block_begin, uint64_t n_blocks,
                           float scale_lo, float scale_hi, void *d_dst,
                           void *stream);

/* ---- VRAM expert-slot cache (RAM -> VRAM tier) --------------------------
 * Replaces the physical VRAM registry of the GPU backend
 * (backend/mod.rs:548-1047: PhysicalGpuExpertRegistry, generation-keyed
 * lookup at :709-741, LRU eviction at :826-840) and the upload half of
 * GpuExpertCache admission (expert_cache.rs:1281-1340).
 *
 * A cache owns an arena of n_slots expert-sized slots in VRAM (expert size
 * = mer_expert_weight_bytes(dtype, d_model, d_ff)), a device table of
 * n_experts pointers (null = not resident) and a copy stream of its own.
 * The table is the expert_table of mer_hip_moe_forward and of
 * mer_layer_args (table_len = n_experts).
 *
 * prepare(ids, generations, host_blobs, n, stream): makes all n experts
 * resident for the work the caller enqueues next on `stream` (its compute
 * stream).  For each id: a stored entry of the same generation is a hit
 * (LRU touch); a newer stored generation fails the call with
 * MER_ERR_RESIDENCY_MISS and changes nothing; an older one is retired and
 * the expert is uploaded from host_blobs[i] (expert-sized; allocate it with
 * mer_hip_host_alloc so the copy overlaps compute) into a free slot or the
 * least recently used slot that this call does not need.  Uploads run on
 * the cache's copy stream; `stream` waits for them (events, no host wait)
 * and then the table entries are written on `stream`.  generations may be
 * NULL (all 0); host_blobs may be NULL or hold NULL for ids known to be
 * resident.  More distinct ids than slots fails with
 * MER_ERR_PHYSICAL_CAPACITY before anything changes.
 *
 * prefetch(...): starts the uploads of misses without making any stream
 * wait and without publishing them (a later prepare does); it never evicts
 * the slots of the last prepare, and ids beyond what then fits are dropped
 * (a prefetch is a hint).  Use it for the predicted experts of the
 * next step (the engine's prefetch hook, engine.rs:5287-5322).
 *
 * A slot is overwritten only after the compute that used it: every prepare
 * and prefetch first records, on `stream`, that the work enqueued there so
 * far may use the last prepare's slots; release() records the same point
 * explicitly (for callers whose compute runs on another stream).  Calls on
 * one cache are serialised by a mutex; `stream` must be the compute stream
 * that uses the table. */
typedef struct mer_slot_cache mer_slot_cache;
typedef struct mer_slot_stats {
  uint64_t hits, misses, prefetches, evictions, stale_retirements;
  uint64_t bytes_uploaded;
  uint64_t resident; /* slots holding an expert now */
} mer_slot_stats;
int mer_slot_cache_create(int dtype, size_t d_model, size_t d_ff, size_t n_slots, size_t n_experts,
                          mer_slot_cache **out);
int mer_slot_cache_destroy(mer_slot_cache *cache);
const void *const *mer_slot_cache_table(mer_slot_cache *cache);
int mer_slot_cache_prepare(mer_slot_cache *cache, const uint32_t *ids, const uint64_t *generations,
                           const void *const *host_blobs, size_t n, void *stream);
int mer_slot_cache_prefetch(mer_slot_cache *cache, const uint32_t *ids, const uint64_t *generations,
                            const void *const *host_blobs, size_t n, void *stream);
int mer_slot_cache_release(mer_slot_cache *cache, void *stream);
int mer_slot_cache_stats(mer_slot_cache *cache, mer_slot_stats *out);
/* Pinned (page-locked) host memory for expert bytes that feed the cache:
 * the RAM tier's page-aligned buffers (expert_cache.rs:55-253) allocated
 * so H2D copies run asynchronously. */
int mer_hip_host_alloc(size_t bytes, void **out);
int mer_hip_host_free(void *p);

/* ---- on-disk expert formats (host only; no device, no mer_hip_init) ----
 * The expert-blob headers and the GGUF reader that feed the RAM tier, so
 * real checkpoints reach the routed forwards byte for byte. */

/* UTH expert-blob headers (tensor_header.rs): a UTH1 (64 B) or UTH2
 * (128 B, per-projection dtype ranges) header at byte 0, optionally padded
 * to the block alignment.  mer_uth_probe strips a blob as
 * ExpertResident::new_with_block_align does (expert_cache.rs:110-143):
 * UTH2 first (probe + range validation), then UTH1, else a headerless
 * (legacy) blob, which is not an error (kind 0, payload = the whole blob). */
typedef struct mer_uth_projection {
  int32_t dtype;   /* UthDtypeId: 4 = Q4_0, 5 = Q8_0, ... */
  uint32_t weights;
  uint64_t offset; /* from the payload start */
  uint64_t len;
} mer_uth_projection;
typedef struct mer_uth_info {
  int32_t kind;              /* 0 headerless, 1 UTH1, 2 UTH2 */
  int32_t dtype;             /* UTH1 dtype id; 10 (mixed) for UTH2; -1 headerless */
  uint32_t version, flags;
  uint32_t shape_rank, shape[4];                  /* UTH1 */
  uint32_t quant_scale_offset, quant_scale_count; /* UTH1 */
  uint32_t d_model, d_ff;    /* UTH2, or a UTH1 SwiGLU expert header [d_ff, d_model, 3] */
  mer_uth_projection proj[3];/* UTH2 gate, up, down */
  uint64_t payload_offset;   /* bytes before the weights */
  uint64_t payload_len;
} mer_uth_info;
int mer_uth_probe(const void *bytes, size_t len, size_t block_align, mer_uth_info *out);
/* TensorHeader::for_swiglu_expert + write_padded (tensor_header.rs:398-470):
 * writes the UTH1 header of a SwiGLU expert blob padded to block_align;
 * *written = the payload offset.  dst = NULL only reports the size. */
int mer_uth_write_expert_header(int dtype, size_t d_model, size_t d_ff, size_t block_align, void *dst,
                                size_t dst_len, size_t *written);

/* GGUF reader for MoE expert tensors (gguf.rs:207-295, gguf_loader.rs:
 * 136-200, :2940-3010): versions 1-3; a layer's experts are either
 * stacked (blk.L.ffn_{gate,up}_exps.weight [d_model, d_ff, E] and
 * blk.L.ffn_down_exps.weight [d_ff, d_model, E], GGML order) or per expert
 * (blk.L.ffn_{gate,up,down}.e.weight).  Only Q4_0 / Q8_0 expert tensors
 * with d_model * d_ff a multiple of 32 are accepted: their expert slices
 * are whole block runs, copied byte for byte into MER's gate || up ||
 * down blob.  Metadata geometry (embedding_length, [expert_]feed_forward_
 * length, expert_count), when present, must agree with the shapes. */
typedef struct mer_gguf mer_gguf;
typedef struct mer_gguf_moe_info {
  int32_t dtype;          /* MER_DTYPE_Q4_0 / MER_DTYPE_Q8_0 */
  int32_t layout;         /* 0 stacked, 1 per-expert tensors */
  uint64_t d_model, d_ff, n_experts;
  uint64_t expert_bytes;  /* mer_expert_weight_bytes(dtype, d_model, d_ff) */
} mer_gguf_moe_info;
int mer_gguf_open(const char *path, mer_gguf **out);
int mer_gguf_close(mer_gguf *g);
int mer_gguf_moe_layer(mer_gguf *g, size_t layer, mer_gguf_moe_info *out);
/* Expert `expert` of `layer` into dst (>= expert_bytes; pinned host memory
 * from mer_hip_host_alloc makes the later upload asynchronous). */
int mer_gguf_read_expert(mer_gguf *g, size_t layer, size_t expert, void *dst, size_t dst_len);

#ifdef __cplusplus
}
#endif
#endif /* MER_HIP_H */
