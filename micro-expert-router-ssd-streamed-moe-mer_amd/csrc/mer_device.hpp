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
// Dot products run on packed integer dot instructions against the input
// vector in block fixed point (see "xq" below).
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

// 64-bit value from two 32-bit halves.  Taking the halves as uint32_t
// matters where they come from __builtin_amdgcn_readfirstlane, which returns
// int: OR-ing that int into a 64-bit value would sign-extend a low half with
// bit 31 set over the high half.
__host__ __device__ constexpr uint64_t join_u32(uint32_t hi, uint32_t lo) { return ((uint64_t)hi << 32) | lo; }

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

// ---------------------------------------------------------------------
// Input vectors in block fixed point ("xq").
//
// Each 32-element block b of an input vector (x for gate/up, h for down) is
// stored as x ~= s_b * x_int with s_b = max|x_b| / (2^22 - 1) and
// |x_int| <= 2^22 - 1 (rounded to nearest): the representation error is at
// most 2^-23 of the block maximum, the size of an f32 rounding of that
// element.  x_int is split into signed digits laid out so that one packed
// integer dot instruction consumes one weight dword:
//   Q4_0: six balanced base-16 digits (-8..7, 4-bit two's complement).
//         Digit plane k, group m (0..3) is a dword whose nibble 2t is the
//         digit of element 4m+t and nibble 2t+1 that of element 4m+16+t --
//         exactly the element order of qs dword m (byte t = qs[4m+t]).
//         dot8(qs_m ^ 0x88888888, plane[k][m]) then sums (q-8)*digit over
//         eight weights (q ^ 8 is q-8 as a 4-bit two's complement value).
//   Q8_0: three balanced base-256 digits (-128..127).  Plane k, group m
//         (0..7): byte t is the digit of element 4m+t; dot4 with the raw
//         int8 weight dword m.
// Per block: 24 digit dwords, index [k * groups + m], plus s_b.
// Balanced digits come for free from offset binary: with
// u = x_int + 0x888888 (resp. 0x808080), digit k = nibble_k(u) ^ 8
// (resp. byte_k(u) ^ 0x80), i.e. the digit-k field of u ^ 0x888888
// (resp. u ^ 0x808080).  Integer accumulation is exact; the three (Q8) or
// six (Q4) per-block digit sums are recombined in f32 once per block.
constexpr int kBlockDigitDwords = 24;
constexpr float kXIntMax = 4194303.0f;  // 2^22 - 1

template <int FMT> struct DigitTraits;
template <> struct DigitTraits<FMT_Q4_0> {
  static constexpr int kGroups = 4;     // groups of 8 elements per block
  static constexpr int kGroupElems = 8;
  static constexpr int kPlanes = 6;
};
template <> struct DigitTraits<FMT_Q8_0> {
  static constexpr int kGroups = 8;     // groups of 4 elements per block
  static constexpr int kGroupElems = 4;
  static constexpr int kPlanes = 3;
};

struct BlockScale {
  float s;    // dequantisation scale of the block (NaN if non-finite input)
  float inv;  // quantisation multiplier
};

__device__ __forceinline__ BlockScale make_block_scale(float amax, bool finite) {
  BlockScale b;
  if (!finite) {
    b.s = __builtin_nanf("");
    b.inv = 0.f;
  } else if (amax == 0.f) {
    b.s = 0.f;
    b.inv = 0.f;
  } else {
    b.s = amax / kXIntMax;
    b.inv = kXIntMax / amax;
  }
  return b;
}

__device__ __forceinline__ int32_t quantize_elem(float v, float inv) {
  float q = __builtin_rintf(v * inv);
  q = __builtin_fminf(__builtin_fmaxf(q, -kXIntMax), kXIntMax);
  return (int32_t)q;
}

// Candle's Q8_0 activation (candle-core 0.10.2 BlockQ8_0::from_float, the
// input side of QMatMul, run_inference_q4_0_qmm, inference.rs:4159-4243):
// d = amax / 127 (amax ignores NaN), inv = d != 0 ? 1/d : 0,
// q = (x * inv).round() as i8 (half away from zero, NaN -> 0, saturating),
// and the block scale is d rounded to f16.  |q| <= 128 needs only digit
// planes 0-2 of the 22-bit layout below; planes 3-5 are zero.
__device__ __forceinline__ BlockScale make_block_scale_q8(float amax) {
  BlockScale b;
  const float d = amax / 127.0f;
  b.inv = d != 0.0f ? 1.0f / d : 0.0f;
  b.s = (float)(_Float16)d;
  return b;
}

__device__ __forceinline__ int32_t quantize_elem_q8(float v, float inv) {
  const float q = __builtin_roundf(v * inv);
  if (__builtin_isnan(q)) return 0;
  return (int32_t)__builtin_fminf(__builtin_fmaxf(q, -128.0f), 127.0f);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t v, int k) { return (v >> (8 * k)) & 0xffu; }

// Element index (within its block) of slot i of group m.
template <int FMT>
__device__ __forceinline__ int group_elem(int m, int i) {
  if constexpr (FMT == FMT_Q4_0) return (i & 1) ? 4 * m + 16 + (i >> 1) : 4 * m + (i >> 1);
  else return 4 * m + i;
}

// Pack one group (8 elements for Q4_0, 4 for Q8_0, in group slot order)
// into its digit-plane dwords: plane[k] goes to digit dword k*groups + m.
// Q8ACT: the values are Candle's Q8_0 activation instead (Q4_0 only).
template <int FMT, bool Q8ACT = false>
__device__ __forceinline__ void pack_group(const float *v, float inv, uint32_t *plane) {
  if constexpr (FMT == FMT_Q4_0) {
    uint32_t t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      t[i] = ((uint32_t)((Q8ACT ? quantize_elem_q8(v[i], inv) : quantize_elem(v[i], inv)) + 0x888888)) ^ 0x888888u;
    uint32_t E[4], O[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = t[2 * j], b = t[2 * j + 1];
      E[j] = (a & 0x0f0f0fu) | ((b << 4) & 0xf0f0f0u);
      O[j] = ((a >> 4) & 0x0f0f0fu) | (b & 0xf0f0f0u);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      plane[2 * k] = byte_of(E[0], k) | (byte_of(E[1], k) << 8) | (byte_of(E[2], k) << 16) | (byte_of(E[3], k) << 24);
      plane[2 * k + 1] = byte_of(O[0], k) | (byte_of(O[1], k) << 8) | (byte_of(O[2], k) << 16) | (byte_of(O[3], k) << 24);
    }
  } else {
    uint32_t t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = ((uint32_t)(quantize_elem(v[i], inv) + 0x808080)) ^ 0x808080u;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      plane[k] = byte_of(t[0], k) | (byte_of(t[1], k) << 8) | (byte_of(t[2], k) << 16) | (byte_of(t[3], k) << 24);
  }
}

// One block's integer dot, recombined to f32: sum_j w_int_j * x_int_j
// with w_int = q-8 (Q4_0) or q (Q8_0).  `q` holds the block's weight dwords
// (4 qs dwords for Q4_0, 8 int8 dwords for Q8_0), `dig` its 24 digit dwords.
// Q8ACT (Q4_0 only): the digits hold a Q8_0 activation in planes 0-2, and
// the block's dot is that one chain, exact in int32.
template <int FMT, bool Q8ACT = false>
__device__ __forceinline__ float block_idot(const uint32_t *q, const uint32_t *dig) {
  if constexpr (FMT == FMT_Q4_0 && Q8ACT) {
    uint32_t qs[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) qs[m] = q[m] ^ 0x88888888u;
    int lo = 0;
#pragma unroll
    for (int k = 2; k >= 0; --k) {
      if (k < 2) lo <<= 4;
#pragma unroll
      for (int m = 0; m < 4; ++m) lo = __builtin_amdgcn_sdot8((int)qs[m], (int)dig[k * 4 + m], lo, false);
    }
    return (float)lo;
  } else if constexpr (FMT == FMT_Q4_0) {
    // Horner over the base-16 planes inside the dot chains: each plane's
    // dots accumulate onto the running sum shifted by 4, so a block needs
    // two zeroed accumulators instead of six.  |plane sum| <= 2048, so
    // planes 0-3 (lo) stay below 2^24 and planes 4-5 (hi) below 2^16.
    uint32_t qs[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) qs[m] = q[m] ^ 0x88888888u;
    int lo = 0, hi = 0;
#pragma unroll
    for (int k = 3; k >= 0; --k) {
      if (k < 3) lo <<= 4;
#pragma unroll
      for (int m = 0; m < 4; ++m) lo = __builtin_amdgcn_sdot8((int)qs[m], (int)dig[k * 4 + m], lo, false);
    }
#pragma unroll
    for (int k = 5; k >= 4; --k) {
      if (k < 5) hi <<= 4;
#pragma unroll
      for (int m = 0; m < 4; ++m) hi = __builtin_amdgcn_sdot8((int)qs[m], (int)dig[k * 4 + m], hi, false);
    }
    return __builtin_fmaf((float)hi, 65536.0f, (float)lo);
  } else {
    // planes 0-1 (|sum| < 2^27) in one chain, plane 2 in another
    int lo = 0, hi = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) lo = __builtin_amdgcn_sdot4((int)q[m], (int)dig[8 + m], lo, false);
    lo <<= 8;
#pragma unroll
    for (int m = 0; m < 8; ++m) lo = __builtin_amdgcn_sdot4((int)q[m], (int)dig[m], lo, false);
#pragma unroll
    for (int m = 0; m < 8; ++m) hi = __builtin_amdgcn_sdot4((int)q[m], (int)dig[16 + m], hi, false);
    return __builtin_fmaf((float)hi, 65536.0f, (float)lo);
  }
}

// Dot of one 64-weight chunk (two blocks) with its input digits.
// dig: 48 dwords (block 0 then block 1), sc: the two block scales.
template <int FMT, bool Q8ACT = false>
__device__ __forceinline__ float chunk_idot(const uint32_t (&w)[FmtTraits<FMT>::kChunkDwords], const uint32_t *dig,
                                            const float *sc) {
  if constexpr (FMT == FMT_Q4_0) {
    const uint32_t q0[4] = {realign16(w[0], w[1]), realign16(w[1], w[2]), realign16(w[2], w[3]),
                            realign16(w[3], w[4])};
    const uint32_t q1[4] = {w[5], w[6], w[7], w[8]};
    const float v0 = block_idot<FMT, Q8ACT>(q0, dig);
    const float v1 = block_idot<FMT, Q8ACT>(q1, dig + kBlockDigitDwords);
    const float d0 = f16_bits_to_f32(w[0] & 0xffffu) * sc[0];
    const float d1 = f16_bits_to_f32(w[4] >> 16) * sc[1];
    return __builtin_fmaf(d1, v1, d0 * v0);
  } else {
    uint32_t q0[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) q0[k] = realign16(w[k], w[k + 1]);
    const float v0 = block_idot<FMT>(q0, dig);
    const float v1 = block_idot<FMT>(&w[9], dig + kBlockDigitDwords);
    const float d0 = f16_bits_to_f32(w[0] & 0xffffu) * sc[0];
    const float d1 = f16_bits_to_f32(w[8] >> 16) * sc[1];
    return __builtin_fmaf(d1, v1, d0 * v0);
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

// SwiGLU element: silu(clamp(g, -limit, limit)) * u.  The clamp is the
// GPT-OSS swiglu_limit (inference.rs:86-123); limit = +inf disables it, and
// a NaN gate stays NaN (as f32::clamp leaves it).
__device__ __forceinline__ float silu_mul(float g, float u, float limit) {
  g = g < -limit ? -limit : (g > limit ? limit : g);
  return g / (1.0f + __expf(-g)) * u;
}

}  // namespace mer
