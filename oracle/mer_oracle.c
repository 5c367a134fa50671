/*
 * mer_oracle.c -- CPU restatement of MER's routed-expert SwiGLU FFN path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Reference paths are relative to rust-engine/src/ of
 * randyap8-wq/Micro-Expert-Router-SSD-Streamed-MoE-MER.
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp).
 * -ffp-contract=off is load-bearing: Rust never fuses a*b+c, so the
 * scalar Q8_0 order (inference.rs:3539-3572) only reproduces bit-for-bit
 * without contraction.  Fused multiply-adds appear only where the
 * reference itself uses _mm256_fmadd_ps (kernels/avx2.rs), via fmaf().
 */
#include "mer_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define Q4_ELEMS 32u
#define Q4_BYTES 18u
#define Q8_ELEMS 32u
#define Q8_BYTES 34u
/* EXPERT_SIZE_TOLERANCE_BYTES = gguf_loader::DEFAULT_BLOCK_ALIGN
 * (inference.rs:3962, gguf_loader.rs:111). */
#define EXPERT_SIZE_TOLERANCE_BYTES 4096u

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Saturating helpers mirroring Rust's saturating_mul / checked_mul. */
static size_t sat_mul(size_t a, size_t b) {
  if (a != 0 && b > SIZE_MAX / a) return SIZE_MAX;
  return a * b;
}
static int checked_mul(size_t a, size_t b, size_t *out) {
  if (a != 0 && b > SIZE_MAX / a) return 0;
  *out = a * b;
  return 1;
}
static size_t div_ceil(size_t a, size_t b) { return a / b + (a % b != 0); }

/* ------------------------------------------------------------------ */
/* f16 <-> f32.  half 2.7.1 (Cargo.lock:1456) to_f32 / from_f32 are the
 * IEEE-754 binary16 conversions (exact widening; round-to-nearest-even
 * narrowing, NaN quieted).  pinned by: tests/test_oracle_golden.py::
 * test_f16_to_f32_exhaustive and ::test_f32_to_f16_matches_numpy.     */
float mo_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1f) /* inf / NaN (NaN quieted, payload kept) */
    return bits_f32(sign | 0x7f800000u | (man ? 0x00400000u : 0) | (man << 13));
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    /* subnormal: man * 2^-24, exact in f32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t mo_f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {
    if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
    return (uint16_t)(sign | 0x7c00u);
  }
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;
    unsigned shift = (unsigned)(14 - e);
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)h;
}

/* Rust `(v).round() as i32`: round half away from zero, then the
 * saturating float->int cast (NaN -> 0). */
int32_t mo_round_to_i32(float v) {
  if (isnan(v)) return 0;
  float r = roundf(v);
  if (r >= 2147483648.0f) return INT32_MAX;
  if (r <= -2147483648.0f) return INT32_MIN;
  return (int32_t)r;
}

static float block_scale(const uint8_t *b) {
  return mo_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
}

/* ------------------------------------------------------------------ */
/* inference.rs:762-784 dequantize_q4_0_block: dst[j] = d*((b&15)-8),
 * dst[j+16] = d*((b>>4)-8).  pinned by: golden ramp/extrema blocks
 * (inference.rs:5613-5637, q4_parity.rs:1429-1440).                  */
void mo_dequantize_q4_0_block(const uint8_t *src, float *dst) {
  float d = block_scale(src);
  for (unsigned j = 0; j < 16; ++j) {
    uint8_t b = src[2 + j];
    dst[j] = d * (float)((int)(b & 0x0f) - 8);
    dst[j + 16] = d * (float)((int)(b >> 4) - 8);
  }
}

/* inference.rs:894-914 dequantize_q8_0_block: dst[i] = d * (i8)q[i]. */
void mo_dequantize_q8_0_block(const uint8_t *src, float *dst) {
  float d = block_scale(src);
  for (unsigned i = 0; i < 32; ++i) dst[i] = d * (float)(int8_t)src[2 + i];
}

/* inference.rs:797-841 quantize_q4_0_block: d = max_abs/7 (f32), stored
 * as f16; zero block stores d=0, nibbles 0x88; q = round(v/d)+8 clamped
 * to 0..15 where the division uses the unrounded f32 d.
 * pinned by: golden writer bytes (inference.rs:5640-5661).            */
void mo_quantize_q4_0_block(const float *src, size_t n, uint8_t *dst) {
  float max_abs = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    float a = fabsf(src[i]);
    if (a > max_abs) max_abs = a;
  }
  float d = max_abs / 7.0f;
  uint16_t db = mo_f32_to_f16(d);
  dst[0] = (uint8_t)(db & 0xff);
  dst[1] = (uint8_t)(db >> 8);
  memset(dst + 2, 0x88, 16);
  if (d == 0.0f) return;
  float inv_d = 1.0f / d;
  for (unsigned j = 0; j < 16; ++j) {
    int32_t q[2];
    for (int h = 0; h < 2; ++h) {
      size_t i = j + 16u * (unsigned)h;
      float v = i < n ? src[i] : 0.0f;
      int32_t r = (int32_t)((uint32_t)mo_round_to_i32(v * inv_d) + 8u);
      q[h] = r < 0 ? 0 : (r > 15 ? 15 : r);
    }
    dst[2 + j] = (uint8_t)(q[0] | (q[1] << 4));
  }
}

/* inference.rs:920-957 quantize_q8_0_block: d = max_abs/127. */
void mo_quantize_q8_0_block(const float *src, size_t n, uint8_t *dst) {
  float max_abs = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    float a = fabsf(src[i]);
    if (a > max_abs) max_abs = a;
  }
  float d = max_abs / 127.0f;
  uint16_t db = mo_f32_to_f16(d);
  dst[0] = (uint8_t)(db & 0xff);
  dst[1] = (uint8_t)(db >> 8);
  if (d == 0.0f) {
    memset(dst + 2, 0, 32);
    return;
  }
  float inv_d = 1.0f / d;
  for (unsigned i = 0; i < 32; ++i) {
    float v = i < n ? src[i] : 0.0f;
    int32_t q = mo_round_to_i32(v * inv_d);
    q = q < -128 ? -128 : (q > 127 ? 127 : q);
    dst[2 + i] = (uint8_t)(int8_t)q;
  }
}

/* inference.rs:852-868 / :963-979: stream decode, tail block truncated. */
int mo_dequantize_to_f32(int dtype, const uint8_t *src, size_t src_len,
                         size_t n_weights, float *dst) {
  size_t bb = dtype == MO_DTYPE_Q4_0 ? Q4_BYTES : Q8_BYTES;
  size_t blocks = div_ceil(n_weights, 32);
  if (src_len < sat_mul(blocks, bb)) return MO_ERR_BUFFER_TOO_SMALL;
  float tmp[32];
  for (size_t b = 0; b < blocks; ++b) {
    if (dtype == MO_DTYPE_Q4_0) mo_dequantize_q4_0_block(src + b * bb, tmp);
    else mo_dequantize_q8_0_block(src + b * bb, tmp);
    size_t n = n_weights - b * 32 < 32 ? n_weights - b * 32 : 32;
    memcpy(dst + b * 32, tmp, n * sizeof(float));
  }
  return MO_OK;
}

/* ------------------------------------------------------------------ */
/* inference.rs:1089-1146 expert_weight_bytes_for: per-tensor block
 * rounding, 3 * ceil(dm*dff/32) * {18,34}, saturating.
 * pinned by: golden sizes 108/216/204 (inference.rs:5748-5758, :5816). */
size_t mo_expert_weight_bytes(int dtype, size_t d_model, size_t d_ff) {
  size_t one = sat_mul(d_model, d_ff);
  size_t blocks = sat_mul(div_ceil(one, 32), 3);
  return sat_mul(blocks, dtype == MO_DTYPE_Q4_0 ? Q4_BYTES : Q8_BYTES);
}

/* inference.rs:1766-1783 + :4035-4077 (strict tolerance semantics). */
int mo_validate_q4_0(size_t len, size_t d_model, size_t d_ff, size_t tolerance,
                     size_t *need_out) {
  size_t n = sat_mul(d_ff, d_model);
  size_t blocks = div_ceil(n, 32);
  size_t need = sat_mul(sat_mul(blocks, 3), Q4_BYTES);
  if (need_out) *need_out = need;
  if (len >= need) return MO_OK;
  if (need > EXPERT_SIZE_TOLERANCE_BYTES &&
      need - len <= EXPERT_SIZE_TOLERANCE_BYTES) {
    if (need - len > tolerance) return MO_ERR_TRUNCATED_PAYLOAD;
    return MO_OK; /* caller zero-pads (non-authoritative legacy mode) */
  }
  return MO_ERR_BUFFER_TOO_SMALL;
}

/* inference.rs:3349-3418 validate_q8_direct_layout. */
int mo_validate_q8_direct(size_t len, size_t x_len, size_t y_len,
                          size_t d_model, size_t d_ff, size_t *need_out) {
  if (need_out) *need_out = 0;
  if (d_model == 0 || d_ff == 0) return MO_ERR_INVALID_LAYOUT;
  if (x_len != d_model || y_len != d_model) return MO_ERR_INVALID_LAYOUT;
  size_t weights, proj, need;
  if (!checked_mul(d_model, d_ff, &weights)) return MO_ERR_INVALID_LAYOUT;
  if (!checked_mul(div_ceil(weights, 32), Q8_BYTES, &proj))
    return MO_ERR_INVALID_LAYOUT;
  if (!checked_mul(proj, 3, &need)) return MO_ERR_INVALID_LAYOUT;
  if (need_out) *need_out = need;
  if (len < need) {
    if (need > EXPERT_SIZE_TOLERANCE_BYTES &&
        need - len <= EXPERT_SIZE_TOLERANCE_BYTES)
      return MO_ERR_TRUNCATED_PAYLOAD;
    return MO_ERR_BUFFER_TOO_SMALL;
  }
  return MO_OK;
}

/* ------------------------------------------------------------------ */
/* Threading: parallel.rs:432-468 par_row_chunks.  Work below 2^18 MACs
 * runs inline; otherwise ntasks = min(threads, total/2^16, rows) chunks
 * of ceil(rows/ntasks) rows.  Each row is computed by exactly one task,
 * so results never depend on the thread count.                        */
#define MIN_TOTAL_FOR_PARALLEL (1u << 18) /* parallel.rs:167 */
#define MIN_ELEMS_PER_TASK (1u << 16)     /* parallel.rs:172 */

typedef void (*row_fn)(void *ctx, size_t row_begin, size_t row_end);

static void par_row_chunks(size_t rows, size_t cols, int nthreads, row_fn f,
                           void *ctx) {
  size_t total = sat_mul(rows, cols ? cols : 1);
  if (rows <= 1 || nthreads <= 1 || total < MIN_TOTAL_FOR_PARALLEL) {
    f(ctx, 0, rows);
    return;
  }
  size_t by_work = total / MIN_ELEMS_PER_TASK;
  if (by_work < 1) by_work = 1;
  size_t ntasks = (size_t)nthreads;
  if (by_work < ntasks) ntasks = by_work;
  if (rows < ntasks) ntasks = rows;
  if (ntasks <= 1) {
    f(ctx, 0, rows);
    return;
  }
  size_t chunk = div_ceil(rows, ntasks);
  size_t nchunks = div_ceil(rows, chunk);
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
  for (size_t c = 0; c < nchunks; ++c) {
    size_t b = c * chunk, e = b + chunk < rows ? b + chunk : rows;
    f(ctx, b, e);
  }
}

/* kernels/avx2.rs:78-87 horizontal_sum_avx2 lane order:
 * ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)).                             */
static float hsum8(const float a[8]) {
  float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
  return (s0 + s1) + (s2 + s3);
}

/* kernels/avx2.rs:35-72 dot_f32_avx2: one 8-lane FMA accumulator,
 * horizontal sum, scalar (non-fused) tail.  This is what
 * kernels::dot_f32 resolves to on an AVX2+FMA host (mod.rs:349-370).  */
static float dot_f32(const float *a, const float *b, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
  float s = hsum8(acc);
  for (; i < n; ++i) s = s + a[i] * b[i];
  return s;
}

/* inference.rs:1630-1634 silu: x / (1 + exp(-x)). */
float mo_silu(float x) { return x / (1.0f + expf(-x)); }

/* inference.rs:86-123: the process-wide GPT-OSS swiglu_limit.
 * set_swiglu_limit keeps a positive finite limit and treats anything else
 * as None (:94-99); clamp_swiglu_gate / the Q8_0 direct path apply
 * g.clamp(-limit, limit) before silu (:118-123, :3699-3701, :3710-3713).
 * f32::clamp leaves NaN as NaN.  pinned by: float64 brute force with the
 * clamp on tiny experts whose gate values straddle the limit
 * (tests/test_oracle_golden.py). */
static float g_swiglu_limit = INFINITY;
void mo_set_swiglu_limit(float limit) {
  g_swiglu_limit = (limit > 0.0f && limit < INFINITY) ? limit : INFINITY;
}
float mo_get_swiglu_limit(void) { return g_swiglu_limit; }
static float clamp_gate(float g) {
  const float l = g_swiglu_limit;
  return g < -l ? -l : (g > l ? l : g);
}

struct gemv_ctx {
  const float *w;
  const float *x;
  float *y;
  size_t cols;
};
static void gemv_rows(void *p, size_t b, size_t e) {
  struct gemv_ctx *c = (struct gemv_ctx *)p;
  for (size_t r = b; r < e; ++r) c->y[r] = dot_f32(c->w + r * c->cols, c->x, c->cols);
}

struct deq_ctx {
  int dtype;
  const uint8_t *src;
  float *dst;
  size_t n_weights;
};
static void deq_rows(void *p, size_t b, size_t e) {
  /* "rows" here are blocks; the tail block is truncated. */
  struct deq_ctx *c = (struct deq_ctx *)p;
  float tmp[32];
  size_t bb = c->dtype == MO_DTYPE_Q4_0 ? Q4_BYTES : Q8_BYTES;
  for (size_t k = b; k < e; ++k) {
    if (c->dtype == MO_DTYPE_Q4_0) mo_dequantize_q4_0_block(c->src + k * bb, tmp);
    else mo_dequantize_q8_0_block(c->src + k * bb, tmp);
    size_t n = c->n_weights - k * 32 < 32 ? c->n_weights - k * 32 : 32;
    memcpy(c->dst + k * 32, tmp, n * sizeof(float));
  }
}

/* Dequantise three per-tensor-rounded projections, then the Candle-style
 * f32 forward: g = W_g x, u = W_u x, h = silu(g)*u, y = W_d h
 * (inference.rs:1442-1473).  Accumulation is f32 in dot_f32 order. */
static int dequant_forward(int dtype, const uint8_t *bytes, const float *x,
                           size_t d_model, size_t d_ff, float *y, int nthreads) {
  size_t n = d_model * d_ff;
  size_t blocks = div_ceil(n, 32);
  size_t bb = dtype == MO_DTYPE_Q4_0 ? Q4_BYTES : Q8_BYTES;
  size_t pb = blocks * bb;
  if (n == 0) {
    for (size_t i = 0; i < d_model; ++i) y[i] = 0.0f;
    return MO_OK;
  }
  float *w = (float *)malloc(sizeof(float) * (blocks * 32) * 3);
  float *g = (float *)malloc(sizeof(float) * d_ff * 2);
  if (!w || !g) {
    free(w);
    free(g);
    return MO_ERR_COMPUTE;
  }
  float *wg = w, *wu = w + blocks * 32, *wd = w + 2 * blocks * 32;
  float *u = g + d_ff;
  struct deq_ctx dc[3] = {{dtype, bytes, wg, n},
                          {dtype, bytes + pb, wu, n},
                          {dtype, bytes + 2 * pb, wd, n}};
  for (int t = 0; t < 3; ++t) par_row_chunks(blocks, 32, nthreads, deq_rows, &dc[t]);
  struct gemv_ctx c1 = {wg, x, g, d_model}, c2 = {wu, x, u, d_model};
  par_row_chunks(d_ff, d_model, nthreads, gemv_rows, &c1);
  par_row_chunks(d_ff, d_model, nthreads, gemv_rows, &c2);
  for (size_t i = 0; i < d_ff; ++i) g[i] = mo_silu(clamp_gate(g[i])) * u[i];
  struct gemv_ctx c3 = {wd, g, y, d_ff};
  par_row_chunks(d_model, d_ff, nthreads, gemv_rows, &c3);
  free(w);
  free(g);
  return MO_OK;
}

/* inference.rs:3291-3306 q4_0_cpu_reference_forward = from_bytes_q4_0
 * (strict) + forward_candle.  pinned by: brute-force float64 forward on
 * small shapes and the q4_parity.rs:1442-1462 fixture.                */
int mo_q4_0_reference_forward(const uint8_t *bytes, size_t len, const float *x,
                              size_t d_model, size_t d_ff, float *y,
                              int nthreads) {
  size_t need;
  int st = mo_validate_q4_0(len, d_model, d_ff, 0, &need);
  if (st != MO_OK) return st;
  return dequant_forward(MO_DTYPE_Q4_0, bytes, x, d_model, d_ff, y, nthreads);
}

/* ------------------------------------------------------------------ */
/* Q4_0 through Candle's QMatMul: run_inference_q4_0_qmm (inference.rs:
 * 4159-4201) -> forward_q4_0_qmm_from_exact_bytes (:4204-4243) ->
 * forward_qmm (:4102-4127), the engine's default Q4_0 arm when both dims
 * are multiples of 32 (use_qmm_for_q4 = true, engine.rs:1144, :1825).
 * The arithmetic lives in candle-core 0.10.2 (Cargo.lock:340-342; a
 * crates.io dependency, not vendored).  Its published quantized CPU matmul
 * converts each activation row to the weight type's vec-dot type, Q8_0 for
 * Q4_0 (k_quants.rs BlockQ8_0::from_float), per 32-element block:
 *   amax = max |x| (f32::max, so NaN is ignored), d = amax / 127,
 *   id = d != 0 ? 1 / d : 0, q = (x * id).round() as i8, d kept as f16;
 * then BlockQ4_0::vec_dot per output row, over the row's blocks in order:
 *   sumi = sum_{j<16} ((w_j & 15) - 8) q_j + ((w_j >> 4) - 8) q_{j+16}
 *   sumf += sumi as f32 * f16(d_w) * f16(d_x).
 * This is that scalar form; Candle's AVX form sums the same integer block
 * dots in another f32 order, so bit-level parity with Candle stays unpinned
 * (the reference pins QMM only to 5e-2 of the dequant path,
 * inference.rs:6547-6594).  The SwiGLU between the projections is
 * forward_qmm's: clamp_swiglu_gate, silu, mul; the down projection
 * quantises h the same way.  pinned by: the reference's own
 * QMM-vs-dequant test (same generator and tolerance), a float64 brute
 * force of the quantisation and dot from the closed forms, and
 * half-way rounding cases (tests/test_oracle_qmm.py).                  */
void mo_quantize_row_q8_0_candle(const float *x, size_t n, int8_t *q, float *d_out) {
  for (size_t b = 0; b < n / 32; ++b) {
    const float *xb = x + b * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
      float a = fabsf(xb[j]);
      if (a > amax) amax = a; /* f32::max: a NaN operand yields the other */
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int j = 0; j < 32; ++j) {
      int32_t v = mo_round_to_i32(xb[j] * id);
      q[b * 32 + j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); /* `as i8` saturates */
    }
    d_out[b] = mo_f16_to_f32(mo_f32_to_f16(d));
  }
}

struct qmm_ctx {
  const uint8_t *w; /* Q4_0 rows of `cols` elements */
  const int8_t *q;  /* Q8_0 activation */
  const float *dq;  /* its block scales */
  float *y;
  size_t cols;
};
static void qmm_rows(void *p, size_t b, size_t e) {
  struct qmm_ctx *c = (struct qmm_ctx *)p;
  size_t nb = c->cols / 32;
  for (size_t r = b; r < e; ++r) {
    const uint8_t *row = c->w + r * nb * Q4_BYTES;
    float sumf = 0.0f;
    for (size_t k = 0; k < nb; ++k) {
      const uint8_t *blk = row + k * Q4_BYTES;
      const int8_t *qb = c->q + k * 32;
      int32_t sumi = 0;
      for (int j = 0; j < 16; ++j) {
        int32_t v0 = (int32_t)(blk[2 + j] & 15) - 8, v1 = (int32_t)(blk[2 + j] >> 4) - 8;
        sumi += v0 * qb[j] + v1 * qb[j + 16];
      }
      sumf += (float)sumi * block_scale(blk) * c->dq[k];
    }
    c->y[r] = sumf;
  }
}

/* Q4_0 weight (r, c) of a row-major projection with `cols` columns. */
static float q4_weight(const uint8_t *proj, size_t cols, size_t r, size_t c) {
  const uint8_t *blk = proj + (r * (cols / 32) + c / 32) * Q4_BYTES;
  unsigned j = (unsigned)(c % 32);
  int nib = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
  return block_scale(blk) * (float)(nib - 8);
}

/* flip_bound (optional, [d_model]): what the down projection's output may
 * move by when another implementation forms h in another f32 order.  An h
 * element whose scaled value h * id lies within `margin` of a rounding
 * midpoint k + 0.5 may round to the neighbouring Q8_0 step there, which
 * moves row r by |W_d[r, j]| * d_j; a block whose d = amax / 127 lies
 * within relative `margin` / 127 of an f16 midpoint may take the
 * neighbouring f16 scale, which moves row r by the block's
 * sum_j |W_d[r, j] q_j| times that f16 step.  *n_flagged counts both. */
int mo_q4_0_qmm_forward_ex(const uint8_t *bytes, size_t len, const float *x, size_t d_model, size_t d_ff, float *y,
                           float *flip_bound, float margin, size_t *n_flagged, int nthreads) {
  size_t need;
  int st = mo_validate_q4_0(len, d_model, d_ff, 0, &need);
  if (st != MO_OK) return st;
  if (d_model % 32 != 0 || d_ff % 32 != 0) return MO_ERR_INVALID_LAYOUT; /* :4211-4215 */
  size_t pb = (d_model * d_ff / 32) * Q4_BYTES;
  size_t big = d_model > d_ff ? d_model : d_ff;
  int8_t *q = (int8_t *)malloc(big);
  float *dq = (float *)malloc(sizeof(float) * (big / 32 + 1));
  float *g = (float *)malloc(sizeof(float) * d_ff * 2);
  if (!q || !dq || !g) {
    free(q);
    free(dq);
    free(g);
    return MO_ERR_COMPUTE;
  }
  float *u = g + d_ff;
  mo_quantize_row_q8_0_candle(x, d_model, q, dq);
  struct qmm_ctx c1 = {bytes, q, dq, g, d_model}, c2 = {bytes + pb, q, dq, u, d_model};
  par_row_chunks(d_ff, d_model, nthreads, qmm_rows, &c1);
  par_row_chunks(d_ff, d_model, nthreads, qmm_rows, &c2);
  for (size_t i = 0; i < d_ff; ++i) g[i] = mo_silu(clamp_gate(g[i])) * u[i];
  mo_quantize_row_q8_0_candle(g, d_ff, q, dq);
  struct qmm_ctx c3 = {bytes + 2 * pb, q, dq, y, d_ff};
  par_row_chunks(d_model, d_ff, nthreads, qmm_rows, &c3);
  if (flip_bound) {
    const uint8_t *wd = bytes + 2 * pb;
    size_t flagged = 0;
    for (size_t r = 0; r < d_model; ++r) flip_bound[r] = 0.0f;
    for (size_t b = 0; b < d_ff / 32; ++b) {
      const float *hb = g + b * 32;
      float amax = 0.0f;
      for (int j = 0; j < 32; ++j) {
        float a = fabsf(hb[j]);
        if (a > amax) amax = a;
      }
      float d = amax / 127.0f;
      float id = d != 0.0f ? 1.0f / d : 0.0f;
      for (int j = 0; j < 32; ++j) {
        float v = hb[j] * id;
        if (!(fabsf(fabsf(v - floorf(v)) - 0.5f) < margin)) continue;
        ++flagged;
        for (size_t r = 0; r < d_model; ++r) flip_bound[r] += fabsf(q4_weight(wd, d_ff, r, b * 32 + j)) * dq[b];
      }
      float lo = mo_f16_to_f32(mo_f32_to_f16(d * (1.0f - margin / 127.0f)));
      float hi = mo_f16_to_f32(mo_f32_to_f16(d * (1.0f + margin / 127.0f)));
      if (lo != hi) {
        ++flagged;
        for (size_t r = 0; r < d_model; ++r) {
          float sum = 0.0f;
          for (int j = 0; j < 32; ++j) sum += fabsf(q4_weight(wd, d_ff, r, b * 32 + j) * (float)q[b * 32 + j]);
          flip_bound[r] += sum * (hi - lo);
        }
      }
    }
    if (n_flagged) *n_flagged = flagged;
  }
  free(q);
  free(dq);
  free(g);
  return MO_OK;
}

int mo_q4_0_qmm_forward(const uint8_t *bytes, size_t len, const float *x, size_t d_model, size_t d_ff, float *y,
                        int nthreads) {
  return mo_q4_0_qmm_forward_ex(bytes, len, x, d_model, d_ff, y, NULL, 0.0f, NULL, nthreads);
}

/* inference.rs:1868-1919 from_bytes_q8_0 + ExpertWeights::forward. */
int mo_q8_0_dequant_forward(const uint8_t *bytes, size_t len, const float *x,
                            size_t d_model, size_t d_ff, float *y,
                            int nthreads) {
  size_t need = mo_expert_weight_bytes(MO_DTYPE_Q8_0, d_model, d_ff);
  if (len < need) return MO_ERR_BUFFER_TOO_SMALL;
  return dequant_forward(MO_DTYPE_Q8_0, bytes, x, d_model, d_ff, y, nthreads);
}

/* ------------------------------------------------------------------ */
/* Native Q8_0 row kernels.
 * kernel 0: inference.rs:3539-3572 scalar order, sum += (d*q)*x.
 * kernel 1: kernels/avx2.rs:98-187, per block w = (float)q * d, then one
 *           FMA per lane into acc[lane][0..8] (lane = 8-element quarter
 *           of the block); acc = (acc0+acc1)+(acc2+acc3); horizontal sum.
 * pinned by: tests comparing both orders against float64 brute force
 * at the reference tolerance (kernels/avx2.rs:224-230, 2e-4+2e-5|r|). */
float mo_q8_0_row_dot(int kernel, const uint8_t *row, const float *x,
                      size_t cols) {
  size_t nb = cols / 32;
  if (kernel == 0) {
    float sum = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t *blk = row + b * Q8_BYTES;
      float s = block_scale(blk);
      for (unsigned i = 0; i < 32; ++i)
        sum = sum + (s * (float)(int8_t)blk[2 + i]) * x[b * 32 + i];
    }
    return sum;
  }
  float acc[4][8];
  memset(acc, 0, sizeof(acc));
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t *blk = row + b * Q8_BYTES;
    float s = block_scale(blk);
    for (int lane = 0; lane < 4; ++lane)
      for (int l = 0; l < 8; ++l) {
        float w = (float)(int8_t)blk[2 + lane * 8 + l] * s;
        acc[lane][l] = fmaf(w, x[b * 32 + lane * 8 + l], acc[lane][l]);
      }
  }
  float t[8];
  for (int l = 0; l < 8; ++l) t[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  return hsum8(t);
}

void mo_q8_0_gate_up_row(int kernel, const uint8_t *g, const uint8_t *u,
                         const float *x, size_t cols, float *gate, float *up) {
  /* The fused traversal (inference.rs:3511-3531, avx2.rs:138-187) keeps
   * separate accumulators per projection, so it equals two row dots. */
  *gate = mo_q8_0_row_dot(kernel, g, x, cols);
  *up = mo_q8_0_row_dot(kernel, u, x, cols);
}

int mo_have_avx2_fma(void) {
#if defined(__x86_64__)
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
  return 0;
#endif
}

/* inference.rs:3618-3632 q8_0_matvec_scalar_flat: flat block stream,
 * blocks may straddle rows. */
static void q8_matvec_flat(const uint8_t *bytes, size_t rows, size_t cols,
                           const float *x, float *y) {
  size_t weights = rows * cols;
  size_t nb = div_ceil(weights, 32);
  for (size_t r = 0; r < rows; ++r) y[r] = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t *blk = bytes + b * Q8_BYTES;
    float s = block_scale(blk);
    size_t base = b * 32;
    size_t count = weights - base < 32 ? weights - base : 32;
    for (size_t i = 0; i < count; ++i) {
      size_t flat = base + i;
      y[flat / cols] = y[flat / cols] + (s * (float)(int8_t)blk[2 + i]) * x[flat % cols];
    }
  }
}

struct q8_ctx {
  int kernel;
  const uint8_t *a, *b;
  const float *x;
  float *out;
  size_t row_bytes, cols;
};
static void q8_gate_up_rows(void *p, size_t b, size_t e) {
  struct q8_ctx *c = (struct q8_ctx *)p;
  for (size_t r = b; r < e; ++r) {
    float g, u;
    mo_q8_0_gate_up_row(c->kernel, c->a + r * c->row_bytes, c->b + r * c->row_bytes,
                        c->x, c->cols, &g, &u);
    c->out[r] = mo_silu(clamp_gate(g)) * u;
  }
}
static void q8_down_rows(void *p, size_t b, size_t e) {
  struct q8_ctx *c = (struct q8_ctx *)p;
  for (size_t r = b; r < e; ++r)
    c->out[r] = mo_q8_0_row_dot(c->kernel, c->a + r * c->row_bytes, c->x, c->cols);
}

/* inference.rs:3659-3746 forward_q8_0_direct_into_with_kernel. */
int mo_q8_0_direct_forward(const uint8_t *bytes, size_t len, const float *x,
                           size_t x_len, size_t d_model, size_t d_ff,
                           float *y, size_t y_len, int kernel, int nthreads) {
  size_t need;
  int st = mo_validate_q8_direct(len, x_len, y_len, d_model, d_ff, &need);
  if (st != MO_OK) return st;
  size_t proj = need / 3;
  const uint8_t *gate = bytes, *up = bytes + proj, *down = bytes + 2 * proj;
  float *h = (float *)malloc(sizeof(float) * d_ff * 2);
  if (!h) return MO_ERR_COMPUTE;
  float *gtmp = h + d_ff;
  if (d_model % 32 == 0) {
    struct q8_ctx c = {kernel, gate, up, x, h, d_model / 32 * Q8_BYTES, d_model};
    par_row_chunks(d_ff, d_model, nthreads, q8_gate_up_rows, &c);
  } else {
    q8_matvec_flat(gate, d_ff, d_model, x, gtmp);
    q8_matvec_flat(up, d_ff, d_model, x, h);
    for (size_t i = 0; i < d_ff; ++i) h[i] = mo_silu(clamp_gate(gtmp[i])) * h[i];
  }
  if (d_ff % 32 == 0) {
    struct q8_ctx c = {kernel, down, NULL, h, y, d_ff / 32 * Q8_BYTES, d_ff};
    par_row_chunks(d_model, d_ff, nthreads, q8_down_rows, &c);
  } else {
    q8_matvec_flat(down, d_model, d_ff, h, y);
  }
  free(h);
  return MO_OK;
}

/* inference.rs:4472-4491 combine_outputs_into: out[j] += s_i * y_i[j] in
 * slot order starting from zero. */
void mo_combine_outputs(const float *outputs, const float *scores, size_t k,
                        size_t d, float *out) {
  for (size_t j = 0; j < d; ++j) out[j] = 0.0f;
  for (size_t i = 0; i < k; ++i)
    for (size_t j = 0; j < d; ++j) out[j] = out[j] + scores[i] * outputs[i * d + j];
}

/* ------------------------------------------------------------------ */
/* inference.rs:3064-3082 synth_hidden_state (splitmix64, top 24 bits). */
void mo_synth_hidden_state(uint64_t token_idx, size_t d_model, uint64_t seed,
                           float *out) {
  uint64_t s = token_idx * 0x9E3779B97F4A7C15ull + seed * 0xBF58476D1CE4E5B9ull;
  for (size_t i = 0; i < d_model; ++i) {
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    uint32_t u = (uint32_t)(z >> 40);
    out[i] = (float)u / 8388608.0f - 1.0f;
  }
}

/* q4_parity.rs:458-466 deterministic_input: ((i*(2s+3)+s) % 31 - 15)/32. */
void mo_deterministic_input(size_t len, size_t seed, float *out) {
  for (size_t i = 0; i < len; ++i) {
    int v = (int)((i * (seed * 2 + 3) + seed) % 31) - 15;
    out[i] = mo_f16_to_f32(mo_f32_to_f16((float)v / 32.0f));
  }
}

/* q4_parity.rs:451-456 canonical_block. */
void mo_canonical_block(float scale, const uint8_t nibbles[16], uint8_t *dst) {
  uint16_t d = mo_f32_to_f16(scale);
  dst[0] = (uint8_t)(d & 0xff);
  dst[1] = (uint8_t)(d >> 8);
  memcpy(dst + 2, nibbles, 16);
}

/* q4_parity.rs:591-653 cpu_q4_matvec + validate_raw_case. */
int mo_cpu_q4_matvec(const uint8_t *weights, size_t weights_len,
                     size_t w_block_off, size_t rows, size_t columns,
                     const float *input, float *out) {
  if (rows == 0 || columns == 0 || columns % 32 != 0) return MO_ERR_INVALID_LAYOUT;
  size_t bpr = columns / 32;
  size_t accessed, required;
  if (!checked_mul(rows, bpr, &accessed)) return MO_ERR_INVALID_LAYOUT;
  if (accessed > SIZE_MAX - w_block_off) return MO_ERR_INVALID_LAYOUT;
  if (!checked_mul(accessed + w_block_off, Q4_BYTES, &required))
    return MO_ERR_INVALID_LAYOUT;
  if (weights_len < required || weights_len % Q4_BYTES != 0)
    return MO_ERR_BUFFER_TOO_SMALL;
  for (size_t i = 0; i < columns; ++i)
    if (!isfinite(input[i])) return MO_ERR_INVALID_LAYOUT;
  float dec[32];
  for (size_t r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (size_t k = 0; k < bpr; ++k) {
      size_t blk = w_block_off + r * bpr + k;
      mo_dequantize_q4_0_block(weights + blk * Q4_BYTES, dec);
      for (size_t c = 0; c < 32; ++c) sum = sum + dec[c] * input[k * 32 + c];
    }
    out[r] = sum;
  }
  return MO_OK;
}

static uint64_t xorshift(uint64_t *s) {
  *s ^= *s << 13;
  *s ^= *s >> 7;
  *s ^= *s << 17;
  return *s;
}

/* inference.rs:5905-5926 randomized_q8_expert (test generator). */
void mo_randomized_q8_expert(size_t d_model, size_t d_ff, uint64_t state,
                             uint8_t *out) {
  size_t weights = d_model * d_ff;
  size_t blocks = div_ceil(weights, 32);
  size_t o = 0;
  for (int p = 0; p < 3; ++p) {
    for (size_t b = 0; b < blocks; ++b) {
      size_t count = weights - b * 32 < 32 ? weights - b * 32 : 32;
      float v[32] = {0};
      for (size_t i = 0; i < count; ++i) {
        xorshift(&state);
        v[i] = ((float)(uint32_t)(state >> 40) / 16777215.0f - 0.5f) *
               (0.08f + (float)p * 0.01f);
      }
      mo_quantize_q8_0_block(v, count, out + o);
      o += Q8_BYTES;
    }
  }
}

/* io_provider.rs:1679-1817 generate_synthetic_experts_with_dtype (Q4_0 /
 * Q8_0 arm): xorshift U(-1,1)/sqrt(d_model), per-tensor block rounding,
 * tail padded with zeros before quantising. */
void mo_generate_synthetic_expert(int dtype, uint32_t id, size_t d_model,
                                  size_t d_ff, uint8_t *out) {
  float scale = 1.0f / sqrtf((float)(d_model ? d_model : 1));
  uint64_t state = 0x9E3779B97F4A7C15ull + (uint64_t)id * 0xBF58476D1CE4E5B9ull;
  size_t one = d_model * d_ff, o = 0;
  size_t bb = dtype == MO_DTYPE_Q4_0 ? Q4_BYTES : Q8_BYTES;
  for (int t = 0; t < 3; ++t) {
    size_t rem = one;
    while (rem > 0) {
      size_t n = rem < 32 ? rem : 32;
      float v[32] = {0};
      for (size_t i = 0; i < n; ++i) {
        xorshift(&state);
        uint32_t u = (uint32_t)(state >> 40);
        v[i] = ((float)u / 8388608.0f - 1.0f) * scale;
      }
      if (dtype == MO_DTYPE_Q4_0) mo_quantize_q4_0_block(v, 32, out + o);
      else mo_quantize_q8_0_block(v, 32, out + o);
      o += bb;
      rem -= n;
    }
  }
}

/* inference.rs:3087-3106 summarise_output: FNV-1a-style digest over the
 * f32 bits, L2 norm in f64. */
uint64_t mo_output_digest(uint64_t token_idx, uint32_t expert_id,
                          const float *y, size_t n, float *norm_out) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)y[i] * (double)y[i];
  if (norm_out) *norm_out = (float)sqrt(ss);
  uint64_t d = 0xcbf29ce484222325ull ^ token_idx ^ (uint64_t)expert_id;
  for (size_t i = 0; i < n; ++i) {
    d ^= (uint64_t)f32_bits(y[i]);
    d *= 0x100000001b3ull;
  }
  return d;
}

/* ------------------------------------------------------------------ */
/* Counter-based bench generator (this build's definition of the
 * synthetic configs: nibbles / int8 values uniform, block scale
 * d = f16(U(lo, hi))).  Block b of expert e owns nine splitmix64
 * finalisations w_i = mix64(seed*G + e*K + 9b + i), i = 0..8:
 *   Q4_0: qs bytes = little-endian bytes of w0, w1; scale from w8.
 *   Q8_0: q[i] = ((16-bit field i of w0..w7) * 255 >> 16) - 127;
 *         scale from w8.
 *   u = (w8 >> 40) / 2^24,  d = f16(lo + (hi - lo) * u).              */
static uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static uint64_t bench_key(uint64_t seed, uint64_t e, uint64_t b) {
  return seed * 0x9E3779B97F4A7C15ull + e * 0xD1B54A32D192ED03ull + 9 * b;
}
static uint16_t bench_scale(uint64_t w8, float lo, float hi) {
  float u = (float)(uint32_t)(w8 >> 40) * (1.0f / 16777216.0f);
  return mo_f32_to_f16(lo + (hi - lo) * u);
}
void mo_bench_fill_q4_0(uint64_t seed, uint64_t expert_index,
                        uint64_t block_begin, uint64_t n_blocks,
                        float scale_lo, float scale_hi, uint8_t *out) {
  for (uint64_t k = 0; k < n_blocks; ++k) {
    uint64_t key = bench_key(seed, expert_index, block_begin + k);
    uint64_t w0 = mix64(key), w1 = mix64(key + 1);
    uint16_t s = bench_scale(mix64(key + 8), scale_lo, scale_hi);
    uint8_t *o = out + k * Q4_BYTES;
    o[0] = (uint8_t)(s & 0xff);
    o[1] = (uint8_t)(s >> 8);
    for (int i = 0; i < 8; ++i) {
      o[2 + i] = (uint8_t)(w0 >> (8 * i));
      o[10 + i] = (uint8_t)(w1 >> (8 * i));
    }
  }
}
void mo_bench_fill_q8_0(uint64_t seed, uint64_t expert_index,
                        uint64_t block_begin, uint64_t n_blocks,
                        float scale_lo, float scale_hi, uint8_t *out) {
  for (uint64_t k = 0; k < n_blocks; ++k) {
    uint64_t key = bench_key(seed, expert_index, block_begin + k);
    uint16_t s = bench_scale(mix64(key + 8), scale_lo, scale_hi);
    uint8_t *o = out + k * Q8_BYTES;
    o[0] = (uint8_t)(s & 0xff);
    o[1] = (uint8_t)(s >> 8);
    for (int w = 0; w < 8; ++w) {
      uint64_t v = mix64(key + (uint64_t)w);
      for (int f = 0; f < 4; ++f) {
        uint32_t v16 = (uint32_t)(v >> (16 * f)) & 0xffffu;
        o[2 + 4 * w + f] = (uint8_t)(int8_t)((int)((v16 * 255u) >> 16) - 127);
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* transformer.rs:2747-2819 softmax_inplace: max over non-NaN entries;
 * NaN or non-finite max -> uniform; else exp(x-max)/sum.              */
void mo_softmax_inplace(float *v, size_t n) {
  if (n == 0) return;
  float max = -INFINITY;
  int saw_nan = 0;
  for (size_t i = 0; i < n; ++i) {
    if (isnan(v[i])) saw_nan = 1;
    else if (v[i] > max) max = v[i];
  }
  if (saw_nan || !isfinite(max)) {
    for (size_t i = 0; i < n; ++i) v[i] = 1.0f / (float)n;
    return;
  }
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    v[i] = expf(v[i] - max);
    sum = sum + v[i];
  }
  if (sum > 0.0f)
    for (size_t i = 0; i < n; ++i) v[i] = v[i] / sum;
}

/* f32::total_cmp key. */
static int32_t total_key(float f) {
  int32_t b;
  memcpy(&b, &f, 4);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* gating.rs:290-339 insert_top_expert + score_id_is_better: higher
 * score first (total order), ties to the lower id; non-finite skipped. */
static void topk_select(const float *scores, size_t n, size_t k, uint32_t *ids,
                        float *sel, size_t *count) {
  size_t c = 0;
  for (size_t e = 0; e < n; ++e) {
    float s = scores[e];
    if (k == 0 || !isfinite(s)) continue;
    size_t pos = c;
    for (size_t i = 0; i < c; ++i) {
      int32_t a = total_key(s), b = total_key(sel[i]);
      if (a > b || (a == b && e < ids[i])) {
        pos = i;
        break;
      }
    }
    if (pos == c && c >= k) continue;
    size_t last = c < k ? c : k - 1;
    for (size_t i = last; i > pos; --i) {
      ids[i] = ids[i - 1];
      sel[i] = sel[i - 1];
    }
    ids[pos] = (uint32_t)e;
    sel[pos] = s;
    if (c < k) c++;
  }
  *count = c;
}

/* gating.rs:395-476 route_with_scratch for the default (Mixtral/Qwen)
 * gate: logits = W x, softmax, top-k, renormalise (sum finite & > 0). */
static size_t route_scores(float *scores, size_t n, size_t top_k, uint32_t *ids,
                           float *weights) {
  mo_softmax_inplace(scores, n);
  float sel[512];
  size_t c = 0;
  float *selp = top_k <= 512 ? sel : (float *)malloc(sizeof(float) * top_k);
  topk_select(scores, n, top_k, ids, selp, &c);
  float sum = 0.0f;
  for (size_t i = 0; i < c; ++i) {
    weights[i] = scores[ids[i]];
    sum = sum + weights[i];
  }
  if (isfinite(sum) && sum > 0.0f)
    for (size_t i = 0; i < c; ++i) weights[i] = weights[i] / sum;
  if (selp != sel) free(selp);
  return c;
}

int mo_linear_gate_route(const float *w, size_t num_experts, size_t d_model,
                         const float *x, size_t top_k, uint32_t *ids,
                         float *weights) {
  float *logits = (float *)malloc(sizeof(float) * num_experts);
  if (!logits) return -1;
  for (size_t e = 0; e < num_experts; ++e)
    logits[e] = dot_f32(w + e * d_model, x, d_model);
  size_t c = route_scores(logits, num_experts, top_k, ids, weights);
  free(logits);
  return (int)c;
}

void mo_topk_softmax_logits(const float *logits, size_t n, size_t top_k,
                            uint32_t *ids, float *weights) {
  float *s = (float *)malloc(sizeof(float) * n);
  memcpy(s, logits, sizeof(float) * n);
  route_scores(s, n, top_k, ids, weights);
  free(s);
}

/* gating.rs:395-476 route_with_scratch, full routing surface
 * (LinearGate::with_routing, gating.rs:207-268):
 *   scores    = softmax(logits) (transformer.rs:2807) or 1/(1+exp(-l))
 *               (gating.rs:271-279);
 *   selection = scores + correction_bias (if any);
 *   optional group filter (gating.rs:332-370): n_group groups of
 *               n/n_group experts scored by the sum of their two best
 *               selection scores (the second only if finite), the best
 *               topk_group groups (score desc by total order, id asc)
 *               survive; disabled unless 1 < topk_group < n_group and
 *               n % n_group == 0 (group_filter_shape, :321-331);
 *   top-k over surviving experts with finite selection scores
 *               (insert_top_expert, :296-320);
 *   weights   = the unbiased scores at the chosen experts, divided by
 *               their (sequential f32) sum when normalise and the sum is
 *               finite and > 0, then multiplied by the routed scaling
 *               factor when it is finite and != 1.
 * pinned by: test_oracle_golden.py (the reference's gating.rs tests:
 * identity-gate sigmoid / bias / group / scaling / tie cases). */
size_t mo_gate_route_ex(const float *logits, size_t n, size_t top_k,
                        int scoring, int normalise, const float *bias,
                        size_t n_group, size_t topk_group, float scaling,
                        uint32_t *ids, float *weights) {
  float *scores = (float *)malloc(sizeof(float) * (n ? n : 1));
  float *selection = (float *)malloc(sizeof(float) * (n ? n : 1));
  uint32_t *gids = (uint32_t *)malloc(sizeof(uint32_t) * (n_group ? n_group : 1));
  float *gsel = (float *)malloc(sizeof(float) * (n_group ? n_group : 1));
  float *tsel = (float *)malloc(sizeof(float) * (top_k ? top_k : 1));
  memcpy(scores, logits, sizeof(float) * n);
  if (scoring == 0) {
    mo_softmax_inplace(scores, n);
  } else {
    for (size_t e = 0; e < n; ++e) scores[e] = 1.0f / (1.0f + expf(-scores[e]));
  }
  for (size_t e = 0; e < n; ++e) selection[e] = bias ? scores[e] + bias[e] : scores[e];
  size_t group_size = 0, n_sel_groups = 0;
  if (n_group > 1 && topk_group > 0 && topk_group < n_group && n % n_group == 0) {
    group_size = n / n_group;
    float *gscore = (float *)malloc(sizeof(float) * n_group);
    for (size_t g = 0; g < n_group; ++g) {
      float top1 = -INFINITY, top2 = -INFINITY;
      for (size_t i = 0; i < group_size; ++i) {
        float v = selection[g * group_size + i];
        if (v > top1) {
          top2 = top1;
          top1 = v;
        } else if (v > top2) {
          top2 = v;
        }
      }
      gscore[g] = top1 + (isfinite(top2) ? top2 : 0.0f);
    }
    /* insert_top_group: total order, lower id on ties, non-finite kept */
    size_t c = 0;
    for (size_t g = 0; g < n_group; ++g) {
      size_t pos = c;
      for (size_t i = 0; i < c; ++i) {
        int32_t a = total_key(gscore[g]), b = total_key(gsel[i]);
        if (a > b || (a == b && g < gids[i])) {
          pos = i;
          break;
        }
      }
      if (pos == c && c >= topk_group) continue;
      size_t last = c < topk_group ? c : topk_group - 1;
      for (size_t i = last; i > pos; --i) {
        gids[i] = gids[i - 1];
        gsel[i] = gsel[i - 1];
      }
      gids[pos] = (uint32_t)g;
      gsel[pos] = gscore[g];
      if (c < topk_group) c++;
    }
    n_sel_groups = c;
    free(gscore);
    /* experts of groups that did not survive cannot be selected */
    for (size_t e = 0; e < n; ++e) {
      int allowed = 0;
      for (size_t i = 0; i < n_sel_groups; ++i)
        if (gids[i] == e / group_size) allowed = 1;
      if (!allowed) selection[e] = NAN; /* skipped as non-finite below */
    }
  }
  size_t cnt = 0;
  topk_select(selection, n, top_k, ids, tsel, &cnt);
  float sum = 0.0f;
  for (size_t i = 0; i < cnt; ++i) {
    weights[i] = scores[ids[i]];
    sum = sum + weights[i];
  }
  if (normalise && isfinite(sum) && sum > 0.0f)
    for (size_t i = 0; i < cnt; ++i) weights[i] = weights[i] / sum;
  if (scaling != 1.0f && isfinite(scaling))
    for (size_t i = 0; i < cnt; ++i) weights[i] = weights[i] * scaling;
  free(scores);
  free(selection);
  free(gids);
  free(gsel);
  free(tsel);
  return cnt;
}

/* logits = W x (dot_f32 order), then mo_gate_route_ex. */
size_t mo_linear_gate_route_ex(const float *w, size_t num_experts, size_t d_model,
                               const float *x, size_t top_k, int scoring,
                               int normalise, const float *bias, size_t n_group,
                               size_t topk_group, float scaling, uint32_t *ids,
                               float *weights, float *logits_out) {
  float *logits = (float *)malloc(sizeof(float) * (num_experts ? num_experts : 1));
  for (size_t e = 0; e < num_experts; ++e)
    logits[e] = dot_f32(w + e * d_model, x, d_model);
  if (logits_out) memcpy(logits_out, logits, sizeof(float) * num_experts);
  size_t c = mo_gate_route_ex(logits, num_experts, top_k, scoring, normalise, bias,
                              n_group, topk_group, scaling, ids, weights);
  free(logits);
  return c;
}

/* ------------------------------------------------------------------ */
/* workload.rs:54-175 SkewedStream. */
struct mo_skewed_stream {
  size_t top_k, n;
  double rho;
  uint32_t *rank_to_id;
  double *cdf;
  uint64_t state;
  uint32_t *prev;
  size_t prev_len;
};

static uint64_t splitmix64(uint64_t *s) {
  *s += 0x9E3779B97F4A7C15ull;
  return mix64(*s);
}
static double next_unit(uint64_t *s) {
  return (double)(splitmix64(s) >> 11) / 9007199254740992.0;
}

mo_skewed_stream *mo_skewed_new(uint32_t num_experts, size_t top_k,
                                double zipf_s, double rho, uint64_t seed) {
  mo_skewed_stream *s = (mo_skewed_stream *)calloc(1, sizeof(*s));
  size_t n = num_experts ? num_experts : 1;
  size_t k = top_k < 1 ? 1 : (top_k > n ? n : top_k);
  double zs = zipf_s > 0.0 ? zipf_s : 0.0;
  s->n = n;
  s->top_k = k;
  s->rho = rho < 0.0 ? 0.0 : (rho > 1.0 ? 1.0 : rho);
  s->cdf = (double *)malloc(sizeof(double) * n);
  double *w = (double *)malloc(sizeof(double) * n);
  double total = 0.0;
  for (size_t r = 0; r < n; ++r) {
    w[r] = 1.0 / pow((double)r + 1.0, zs);
    total += w[r];
  }
  double acc = 0.0;
  for (size_t r = 0; r < n; ++r) {
    acc += w[r] / total;
    s->cdf[r] = acc;
  }
  s->cdf[n - 1] = 1.0;
  free(w);
  uint64_t ps = seed ^ 0xD1B54A32D192ED03ull;
  s->rank_to_id = (uint32_t *)malloc(sizeof(uint32_t) * n);
  for (size_t i = 0; i < n; ++i) s->rank_to_id[i] = (uint32_t)i;
  for (size_t i = n - 1; i >= 1; --i) {
    size_t j = (size_t)(splitmix64(&ps) % ((uint64_t)i + 1));
    uint32_t t = s->rank_to_id[i];
    s->rank_to_id[i] = s->rank_to_id[j];
    s->rank_to_id[j] = t;
  }
  s->state = seed + 0x12345678ull;
  s->prev = (uint32_t *)malloc(sizeof(uint32_t) * k);
  s->prev_len = 0;
  return s;
}

static size_t sample_rank(const mo_skewed_stream *s, double u) {
  /* binary_search_by(total_cmp): first index with cdf >= u (cdf values
   * are distinct), clamped to the last rank. */
  size_t lo = 0, hi = s->n;
  while (lo < hi) {
    size_t mid = lo + (hi - lo) / 2;
    if (s->cdf[mid] < u) lo = mid + 1;
    else hi = mid;
  }
  return lo < s->n ? lo : s->n - 1;
}

static int contains(const uint32_t *v, size_t n, uint32_t x) {
  for (size_t i = 0; i < n; ++i)
    if (v[i] == x) return 1;
  return 0;
}

size_t mo_skewed_next(mo_skewed_stream *s, uint32_t *out) {
  if (s->prev_len && next_unit(&s->state) < s->rho) {
    memcpy(out, s->prev, s->prev_len * sizeof(uint32_t));
    return s->prev_len;
  }
  size_t c = 0, guard = 0;
  size_t guard_max = s->top_k * 64 > 64 ? s->top_k * 64 : 64;
  while (c < s->top_k && guard < guard_max) {
    double u = next_unit(&s->state);
    uint32_t id = s->rank_to_id[sample_rank(s, u)];
    if (!contains(out, c, id)) out[c++] = id;
    guard++;
  }
  for (size_t r = 0; c < s->top_k && r < s->n; ++r) {
    uint32_t id = s->rank_to_id[r];
    if (!contains(out, c, id)) out[c++] = id;
  }
  memcpy(s->prev, out, c * sizeof(uint32_t));
  s->prev_len = c;
  return c;
}

void mo_skewed_free(mo_skewed_stream *s) {
  if (!s) return;
  free(s->rank_to_id);
  free(s->cdf);
  free(s->prev);
  free(s);
}
