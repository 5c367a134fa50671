/*
 * mer_oracle.h -- CPU restatement of MER's routed-expert SwiGLU FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * product path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library never links it and
 * has no CPU fallback through it.
 *
 * Every function cites the reference file:line it restates (paths are
 * relative to rust-engine/src/ of the reference).  Pinning of each
 * function (golden vectors / closed forms / brute force) is recorded
 * next to it as "pinned by: <test>".
 */
#ifndef MER_ORACLE_H
#define MER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes are the same numeric values the product C-ABI uses
 * (include/mer_hip.h) so tests can compare error taxonomies directly. */
enum {
  MO_OK = 0,
  MO_ERR_BUFFER_TOO_SMALL = 1,
  MO_ERR_MISALIGNED = 2,
  MO_ERR_COMPUTE = 3,
  MO_ERR_INVALID_LAYOUT = 4,
  MO_ERR_TRUNCATED_PAYLOAD = 5,
};

enum { MO_DTYPE_Q4_0 = 4, MO_DTYPE_Q8_0 = 5 };

/* ---- scalar conversions ------------------------------------------- */
float mo_f16_to_f32(uint16_t h);              /* half::f16::to_f32        */
uint16_t mo_f32_to_f16(float f);              /* half::f16::from_f32 (RNE) */
int32_t mo_round_to_i32(float v);             /* (v.round()) as i32        */

/* ---- block formats (inference.rs:725-979) -------------------------- */
void mo_dequantize_q4_0_block(const uint8_t *src, float *dst);
void mo_dequantize_q8_0_block(const uint8_t *src, float *dst);
void mo_quantize_q4_0_block(const float *src, size_t n, uint8_t *dst);
void mo_quantize_q8_0_block(const float *src, size_t n, uint8_t *dst);
int mo_dequantize_to_f32(int dtype, const uint8_t *src, size_t src_len,
                         size_t n_weights, float *dst);

/* ---- sizing and validation ----------------------------------------- */
size_t mo_expert_weight_bytes(int dtype, size_t d_model, size_t d_ff);
int mo_validate_q4_0(size_t len, size_t d_model, size_t d_ff, size_t tolerance,
                     size_t *need_out);
int mo_validate_q8_direct(size_t len, size_t x_len, size_t y_len,
                          size_t d_model, size_t d_ff, size_t *need_out);

/* ---- expert forward ----------------------------------------------- */
/* Candle QMatMul Q4_0 path (activations quantised to Q8_0). */
void mo_quantize_row_q8_0_candle(const float *x, size_t n, int8_t *q, float *d_out);
int mo_q4_0_qmm_forward(const uint8_t *bytes, size_t len, const float *x, size_t d_model, size_t d_ff, float *y,
                        int nthreads);
int mo_q4_0_qmm_forward_ex(const uint8_t *bytes, size_t len, const float *x, size_t d_model, size_t d_ff, float *y,
                           float *flip_bound, float margin, size_t *n_flagged, int nthreads);
int mo_q4_0_reference_forward(const uint8_t *bytes, size_t len, const float *x,
                              size_t d_model, size_t d_ff, float *y,
                              int nthreads);
int mo_q8_0_dequant_forward(const uint8_t *bytes, size_t len, const float *x,
                            size_t d_model, size_t d_ff, float *y,
                            int nthreads);
/* kernel: 0 = scalar order, 1 = AVX2 lane order (4x8 FMA accumulators) */
int mo_q8_0_direct_forward(const uint8_t *bytes, size_t len, const float *x,
                           size_t x_len, size_t d_model, size_t d_ff,
                           float *y, size_t y_len, int kernel, int nthreads);
float mo_q8_0_row_dot(int kernel, const uint8_t *row, const float *x,
                      size_t cols);
void mo_q8_0_gate_up_row(int kernel, const uint8_t *g, const uint8_t *u,
                         const float *x, size_t cols, float *gate, float *up);
int mo_have_avx2_fma(void);
void mo_set_swiglu_limit(float limit);
float mo_get_swiglu_limit(void);
float mo_silu(float x);
void mo_combine_outputs(const float *outputs, const float *scores, size_t k,
                        size_t d, float *out);

/* ---- fixtures / generators ---------------------------------------- */
void mo_synth_hidden_state(uint64_t token_idx, size_t d_model, uint64_t seed,
                           float *out);
void mo_deterministic_input(size_t len, size_t seed, float *out);
void mo_canonical_block(float scale, const uint8_t nibbles[16], uint8_t *dst);
int mo_cpu_q4_matvec(const uint8_t *weights, size_t weights_len,
                     size_t w_block_off, size_t rows, size_t columns,
                     const float *input, float *out);
void mo_randomized_q8_expert(size_t d_model, size_t d_ff, uint64_t state,
                             uint8_t *out);
void mo_generate_synthetic_expert(int dtype, uint32_t id, size_t d_model,
                                  size_t d_ff, uint8_t *out);
uint64_t mo_output_digest(uint64_t token_idx, uint32_t expert_id,
                          const float *y, size_t n, float *norm_out);

/* Counter-based synthetic bench generator (this build's definition; the
 * HIP library carries the same generator and parity-tests against it). */
void mo_bench_fill_q4_0(uint64_t seed, uint64_t expert_index,
                        uint64_t block_begin, uint64_t n_blocks,
                        float scale_lo, float scale_hi, uint8_t *out);
void mo_bench_fill_q8_0(uint64_t seed, uint64_t expert_index,
                        uint64_t block_begin, uint64_t n_blocks,
                        float scale_lo, float scale_hi, uint8_t *out);

/* ---- routing (gating.rs, workload.rs) ------------------------------ */
void mo_softmax_inplace(float *v, size_t n);
int mo_linear_gate_route(const float *w, size_t num_experts, size_t d_model,
                         const float *x, size_t top_k, uint32_t *ids,
                         float *weights);
/* Full LinearGate routing surface (gating.rs:207-476): scoring 0 = softmax,
 * 1 = sigmoid; bias may be NULL; returns the number of experts chosen. */
size_t mo_gate_route_ex(const float *logits, size_t n, size_t top_k,
                        int scoring, int normalise, const float *bias,
                        size_t n_group, size_t topk_group, float scaling,
                        uint32_t *ids, float *weights);
size_t mo_linear_gate_route_ex(const float *w, size_t num_experts, size_t d_model,
                               const float *x, size_t top_k, int scoring,
                               int normalise, const float *bias, size_t n_group,
                               size_t topk_group, float scaling, uint32_t *ids,
                               float *weights, float *logits_out);
void mo_topk_softmax_logits(const float *logits, size_t n, size_t top_k,
                            uint32_t *ids, float *weights);

typedef struct mo_skewed_stream mo_skewed_stream;
mo_skewed_stream *mo_skewed_new(uint32_t num_experts, size_t top_k,
                                double zipf_s, double rho, uint64_t seed);
size_t mo_skewed_next(mo_skewed_stream *s, uint32_t *out);
void mo_skewed_free(mo_skewed_stream *s);

#ifdef __cplusplus
}
#endif
#endif
