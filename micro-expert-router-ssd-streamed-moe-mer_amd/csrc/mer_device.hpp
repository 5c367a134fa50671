// mer_device.hpp -- GGUF Q4_0 / Q8_0 block decoding for gfx950 kernels.
//
// Block formats (reference inference.rs:725-979):
//   Q4_0: 18 B = f16 d (LE) + 16 B qs; element j = qs[j] & 15, element
//         j+16 = qs[j] >> 4, value d * (q - 8).
//   Q8_0: 34 B = f16 d (LE) + 32 x int8, value d * q.
//
// The streaming kernels read a row as 64-weight "chunks" (two blocks):
// 36 B for Q4_0 and 68 B for Q8_0.  Whenever a row holds an even number of
// blocks, every chunk starts 4-byte aligned, so a lane fetches its chunk
// with dwordx4 loads (gfx950 accepts 4-byte aligned dwordx4 on global
// memory) and re-splits the blocks in registers:
//   Q4_0 chunk dwords w0..w8: block0 d = w0[15:0], qs = bytes 2..17
//     (realigned from w0..w4 with alignbit); block1 d = w4[31:16],
//     qs = w5..w8.
//   Q8_0 chunk dwords w0..w16: block0 d = w0[15:0], q = bytes 2..33
//     (realigned from w0..w8); block1 d = w8[31:16], q = w9..w16.
//
// Dot products avoid a per-weight subtract: a block contributes
//   Q4_0: d * (sum_j q_j x_j - 8 * sum_j x_j)          q_j in 0..15
//   Q8_0: d * (sum_j u_j x_j - 128 * sum_j x_j)        u_j = q_j + 128
// where each integer converts to f32 with one v_cvt_f32_ubyteN.  High
// Q4 nibbles are used in place (byte & 0xF0 == 16 q) against x/16, which
// is exact in binary floating point.  The per-block input sums are
// computed once per lane and reused for every row the lane visits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mer {

enum Fmt : int { FMT_Q4_0 = 0, FMT_Q8_0 = 1 };

template <int FMT> struct FmtTraits;
template <> struct FmtTraits<FMT_Q4_0> {
  static constexpr int kBlockBytes = 18;
  static constexpr int kChunkBytes = 36;
  static constexpr int kChunkDwords = 9;
};
template <> struct FmtTraits<FMT_Q8_0> {
  static constexpr int kBlockBytes = 34;
  static constexpr int kChunkBytes = 68;
  static constexpr int kChunkDwords = 17;
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// IEEE binary16 -> binary32 (exact), as half::f16::to_f32.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v;
  uint16_t b = (uint16_t)h;
  __builtin_memcpy(&v, &b, 2);
  return (float)v;
}

// binary32 -> binary16 bits, round to nearest even (half::f16::from_f32).
__host__ __device__ inline uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  __builtin_memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | (man ? (0x7e00u | (man >> 13)) : 0x7c00u));
  int e = (int)exp - 112;
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

__device__ __forceinline__ uint32_t realign16(uint32_t lo, uint32_t hi) {
  // bytes 2..5 of the little-endian pair (lo, hi)
  return __builtin_amdgcn_alignbit(hi, lo, 16);
}

template <int FMT>
__device__ __forceinline__ void load_chunk(const uint8_t *p, uint32_t (&w)[FmtTraits<FMT>::kChunkDwords]) {
  const u32x4a4 *v = reinterpret_cast<const u32x4a4 *>(p);
  constexpr int kVec = FmtTraits<FMT>::kChunkDwords / 4;
#pragma unroll
  for (int i = 0; i < kVec; ++i) {
    u32x4a4 a = v[i];
    w[4 * i + 0] = a.x;
    w[4 * i + 1] = a.y;
    w[4 * i + 2] = a.z;
    w[4 * i + 3] = a.w;
  }
  w[4 * kVec] = reinterpret_cast<const uint32_t *>(p)[4 * kVec];
}

// Per-lane copy of the input slice for one chunk, pre-transformed.
//   Q4_0: xv[b*32 + j]      = x[j]        (j < 16, low nibbles)
//         xv[b*32 + 16 + j] = x[16+j]/16  (high nibbles used as 16 q)
//         bias[b] = 8 * sum(x over block b)
//   Q8_0: xv = x, bias[b] = 128 * sum(x over block b)
template <int FMT> struct XSlice {
  float xv[64];
  float bias[2];
};

template <int FMT>
__device__ __forceinline__ void load_xslice(const float *x, XSlice<FMT> &s) {
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float4 v = x4[i];
    s.xv[4 * i + 0] = v.x;
    s.xv[4 * i + 1] = v.y;
    s.xv[4 * i + 2] = v.z;
    s.xv[4 * i + 3] = v.w;
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) sum += s.xv[b * 32 + j];
    s.bias[b] = (FMT == FMT_Q4_0 ? 8.f : 128.f) * sum;
    if (FMT == FMT_Q4_0) {
#pragma unroll
      for (int j = 16; j < 32; ++j) s.xv[b * 32 + j] *= 0.0625f;
    }
  }
}

template <int FMT>
__device__ __forceinline__ void zero_xslice(XSlice<FMT> &s) {
#pragma unroll
  for (int i = 0; i < 64; ++i) s.xv[i] = 0.f;
  s.bias[0] = s.bias[1] = 0.f;
}

__device__ __forceinline__ float fma_bytes(uint32_t u, const float *x, float a) {
  a = __builtin_fmaf((float)(u & 0xffu), x[0], a);
  a = __builtin_fmaf((float)((u >> 8) & 0xffu), x[1], a);
  a = __builtin_fmaf((float)((u >> 16) & 0xffu), x[2], a);
  a = __builtin_fmaf((float)(u >> 24), x[3], a);
  return a;
}

// sum_j q_j x_j over one Q4_0 block given its four qs dwords.
__device__ __forceinline__ float q4_block_raw(const uint32_t (&q)[4], const float *xv) {
  float a = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a = fma_bytes(q[k] & 0x0f0f0f0fu, xv + 4 * k, a);
    a = fma_bytes(q[k] & 0xf0f0f0f0u, xv + 16 + 4 * k, a);
  }
  return a;
}

template <int FMT>
__device__ __forceinline__ float chunk_dot(const uint32_t (&w)[FmtTraits<FMT>::kChunkDwords],
                                           const XSlice<FMT> &s) {
  if constexpr (FMT == FMT_Q4_0) {
    const float d0 = f16_bits_to_f32(w[0] & 0xffffu);
    const float d1 = f16_bits_to_f32(w[4] >> 16);
    uint32_t q0[4] = {realign16(w[0], w[1]), realign16(w[1], w[2]), realign16(w[2], w[3]),
                      realign16(w[3], w[4])};
    uint32_t q1[4] = {w[5], w[6], w[7], w[8]};
    float a0 = q4_block_raw(q0, s.xv);
    float a1 = q4_block_raw(q1, s.xv + 32);
    return __builtin_fmaf(d1, a1 - s.bias[1], d0 * (a0 - s.bias[0]));
  } else {
    const float d0 = f16_bits_to_f32(w[0] & 0xffffu);
    const float d1 = f16_bits_to_f32(w[8] >> 16);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      a0 = fma_bytes(realign16(w[k], w[k + 1]) ^ 0x80808080u, s.xv + 4 * k, a0);
      a1 = fma_bytes(w[9 + k] ^ 0x80808080u, s.xv + 32 + 4 * k, a1);
    }
    return __builtin_fmaf(d1, a1 - s.bias[1], d0 * (a0 - s.bias[0]));
  }
}

// Generic element access for the flat (block-straddling) layout.
template <int FMT>
__device__ __forceinline__ float flat_weight(const uint8_t *proj, size_t flat) {
  const size_t blk = flat >> 5;
  const unsigned j = (unsigned)(flat & 31u);
  const uint8_t *b = proj + blk * FmtTraits<FMT>::kBlockBytes;
  const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
  if constexpr (FMT == FMT_Q4_0) {
    const uint8_t byte = b[2 + (j & 15u)];
    const int q = j < 16 ? (byte & 0x0f) : (byte >> 4);
    return d * (float)(q - 8);
  } else {
    return d * (float)(int8_t)b[2 + j];
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

}  // namespace mer
