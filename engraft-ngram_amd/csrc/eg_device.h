// Device-side building blocks shared by the gfx950 kernels of the n-gram table
// path: the row hash, the unsigned 64-by-32-bit modulus, row-format decoders
// and rounding helpers.  Everything here is integer or exact fp32 arithmetic, so
// the kernels reproduce the CPU definitions bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "engraft_ngram.h"

namespace eg {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Hash parameters as a kernel argument.
// ---------------------------------------------------------------------------
struct LayerHash {
  uint64_t eos;
  int32_t ngram_size;
  int32_t heads_per_ngram;
  int32_t n_heads;
  int32_t pad_;
  uint64_t mult[EG_MAX_NGRAM];       // shared multipliers (reference mode)
  const uint64_t* head_mult;         // device [n_heads][ngram_size] or nullptr
  uint64_t magic[EG_MAX_HEADS];      // floor((2^64 - 1) / vocab[h])
  uint32_t vocab[EG_MAX_HEADS];
  int32_t offset[EG_MAX_HEADS];
};

// x mod p for p in [1, 2^32).  magic = floor((2^64-1)/p) gives
// q = floor(x*magic / 2^64) in [floor(x/p) - 2, floor(x/p)], so the remainder
// x - q*p lies in [0, 3p): at most two corrections.
__host__ __device__ inline uint32_t fastmod_u64(uint64_t x, uint32_t p, uint64_t magic) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint64_t q = __umul64hi(x, magic);
#else
  uint64_t q = (uint64_t)(((unsigned __int128)x * magic) >> 64);
#endif
  uint64_t r = x - q * (uint64_t)p;
  if (r >= p) r -= p;
  if (r >= p) r -= p;
  return (uint32_t)r;
}

// Raw tokens x_t, x_{t-1}, ... of position p (indices clamped at 0; slots
// before the segment start are discarded by ctx_from).  Loading them apart from
// their use lets a kernel issue them before its bulk loads: vmcnt retires
// vector memory operations in order, so a wait for the tokens then does not
// wait for the bulk data.
template <typename TOK>
__device__ inline void load_ctx_tokens(const TOK* __restrict__ tokens, int64_t p, int ngram_size,
                                       uint64_t raw[EG_MAX_NGRAM]) {
#pragma unroll
  for (int s = 0; s < EG_MAX_NGRAM; ++s) {
    raw[s] = 0;
    if (s < ngram_size) {
      const int64_t pos = p - s;
      raw[s] = (uint64_t)tokens[pos < 0 ? 0 : pos];
    }
  }
}

// ctx = [x_t, x_{t-1}, ...]: a predecessor before the segment start, or an EOS
// met while walking back, sets its slot and every older slot to the EOS id; the
// current token's own EOS does not cut (engraft/table.py:121-131).
__device__ inline void ctx_from(const LayerHash& L, const uint64_t raw[EG_MAX_NGRAM], int64_t p, int64_t seg0,
                                uint64_t ctx[EG_MAX_NGRAM]) {
  ctx[0] = raw[0];
  bool cut = false;
#pragma unroll
  for (int s = 1; s < EG_MAX_NGRAM; ++s) {
    uint64_t tok = L.eos;
    if (s < L.ngram_size) {
      const bool valid = !cut && p - s >= seg0;
      if (valid) tok = raw[s];
      if (!valid || tok == L.eos) {
        cut = true;
        tok = L.eos;
      }
    }
    ctx[s] = tok;
  }
}

template <typename TOK>
__device__ inline void build_ctx(const LayerHash& L, const TOK* __restrict__ tokens, int64_t p, int64_t seg0,
                                 uint64_t ctx[EG_MAX_NGRAM]) {
  uint64_t raw[EG_MAX_NGRAM];
  load_ctx_tokens(tokens, p, L.ngram_size, raw);
  ctx_from(L, raw, p, seg0, ctx);
}

// Multipliers of head h (loaded ahead of use like the tokens).
__device__ inline void load_head_mult(const LayerHash& L, int h, uint64_t m[EG_MAX_NGRAM]) {
#pragma unroll
  for (int j = 0; j < EG_MAX_NGRAM; ++j) {
    m[j] = L.mult[j];
    if (L.head_mult && j < L.ngram_size) m[j] = L.head_mult[(int64_t)h * L.ngram_size + j];
  }
}

// The modulus constants of head h (kernel-argument arrays indexed per lane are
// memory loads: a kernel loads them ahead of use, like the multipliers).
struct HeadConst {
  uint64_t magic;
  uint32_t vocab;
  int32_t offset;
};

__device__ inline HeadConst load_head_const(const LayerHash& L, int h) {
  return HeadConst{L.magic[h], L.vocab[h], L.offset[h]};
}

// Global (or local) row of head h from its context, multipliers and constants.
__device__ inline int32_t row_of(const LayerHash& L, int h, const uint64_t ctx[EG_MAX_NGRAM],
                                 const uint64_t m[EG_MAX_NGRAM], const HeadConst& hc, bool global_ids) {
  const int order = 2 + h / L.heads_per_ngram;
  uint64_t mixed = 0;
#pragma unroll
  for (int j = 0; j < EG_MAX_NGRAM; ++j)
    if (j < order) mixed ^= ctx[j] * m[j];
  const uint32_t local = fastmod_u64(mixed, hc.vocab, hc.magic);
  return global_ids ? hc.offset + (int32_t)local : (int32_t)local;
}

// Global row of head h: offset + (XOR_{j<order} ctx[j]*m[j]) mod vocab.
__device__ inline int32_t head_row(const LayerHash& L, int h, const uint64_t ctx[EG_MAX_NGRAM],
                                   bool global_ids) {
  uint64_t m[EG_MAX_NGRAM];
  load_head_mult(L, h, m);
  return row_of(L, h, ctx, m, load_head_const(L, h), global_ids);
}

// Segment start of flat position p.
// (A caller-supplied start below 0 is read as 0: the hash never reads before
// the token array.)
__device__ inline int64_t seg_start_of(int64_t p, int64_t seq_len, const int32_t* seg_start) {
  if (seg_start) return seg_start[p] < 0 ? 0 : seg_start[p];
  if (seq_len > 0) return (p / seq_len) * seq_len;
  return 0;
}

// ---------------------------------------------------------------------------
// Number formats
// ---------------------------------------------------------------------------
__device__ inline float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Round to nearest even; NaN stays a quiet NaN.
__host__ __device__ inline uint32_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t u = __float_as_uint(f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
#endif
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 values to bf16 packed lo | hi << 16, in one gfx950
// v_cvt_pk_bf16_f32 (round to nearest even, NaN quieted): bit-identical to
// f32_to_bf16 on all 2^32 fp32 inputs (checked exhaustively on an MI355X).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ inline float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}

__device__ inline uint16_t f32_to_f16(float f) {
  _Float16 v = (_Float16)f;  // round to nearest even
  return __builtin_bit_cast(uint16_t, v);
}

// OCP e4m3 (float8_e4m3fn): bias 7, subnormals m*2^-9, 0x7f/0xff NaN.  gfx950's
// v_cvt_pk_f32_fp8 converts two such bytes exactly (every code is checked
// against the definition); byte 0 of b here.
__device__ inline float e4m3_to_f32(uint32_t b) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false)[0]; }

// The four e4m3 bytes of w, byte 0 first.
__device__ inline void e4m3x4_to_f32(uint32_t w, float out[4]) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);  // bytes 0, 1
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);   // bytes 2, 3
  out[0] = lo[0];
  out[1] = lo[1];
  out[2] = hi[0];
  out[3] = hi[1];
}

// e8m0 scale 2^(e-127); 0xff is NaN.
__device__ inline float e8m0_to_f32(uint32_t e) {
  if (e == 0xffu) return __uint_as_float(0x7fc00000u);
  if (e == 0) return __uint_as_float(0x00400000u);  // 2^-127 (subnormal)
  return __uint_as_float(e << 23);
}

// RNE fp32 -> e4m3 for |x| <= 448 (callers clamp); the sign bit is kept.
__device__ inline uint32_t f32_to_e4m3(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0.015625f) {                      // below 2^-6: subnormal grid m*2^-9
    code = (uint32_t)rintf(a * 512.0f);     // 0..8; 8 is the smallest normal
  } else {
    int e = (int)((__float_as_uint(a) >> 23) & 0xffu) - 127;  // floor(log2 a), -6..8
    const float mant = __uint_as_float((__float_as_uint(a) & 0x807fffffu) | 0x3f800000u);
    uint32_t m = (uint32_t)rintf((mant - 1.0f) * 8.0f);
    if (m == 8u) { m = 0u; ++e; }
    code = ((uint32_t)(e + 7) << 3) | m;
  }
  return code | sign;
}

// IQ4_NL codebook (GGML kvalues_iq4nl; engraft/table.py:26-29):
//   -127 -104 -83 -65 -49 -35 -22 -10 1 13 25 38 53 69 89 113
// held in registers as int8 bytes.  iq4nl_lookup4 maps four nibbles at once
// (one per byte of n, each < 16) to four int8 codebook bytes: v_perm_b32 picks
// bytes of a 64-bit pair by a 3-bit index, and bit 3 chooses the half.
__device__ inline uint32_t iq4nl_lookup4(uint32_t n) {
  const uint32_t sel = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);  // kvalues[0..7]
  const uint32_t hi = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);  // kvalues[8..15]
  const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;
  return (hi & m) | (lo & ~m);
}

__device__ inline float iq4nl_value(uint32_t nib) { return (float)(int8_t)(iq4nl_lookup4(nib & 15u) & 0xffu); }

// ---------------------------------------------------------------------------
// Row chunk loads: 8 consecutive values [off, off+8) of a row, dequantised to
// fp32.  off is a multiple of 8, so a chunk never straddles a 32-value block.
// ---------------------------------------------------------------------------
struct TableDev {
  const uint8_t* payload;
  const uint8_t* scales;
  int64_t n_rows;
  int32_t fmt;
  int32_t dim;
  int64_t stride;  // IQ4_NL: bytes from one row to the next (its 18-byte blocks, or padded lines)
};

// Raw bytes of one chunk, loaded apart from their decoding so that a kernel can
// issue every load before it waits for any.
struct RawChunk {
  u32x4 w0;     // payload words (BF16: 8 values; Q8_0/MXFP8: .xy; IQ4_NL: 4 nibble halfwords)
  u32x4 w1;     // F32 only: values 4..7
  uint32_t s;   // scale bits (Q8_0/IQ4_NL: fp16; MXFP8: e8m0)
};

template <int FMT>
__device__ inline RawChunk load_raw(const TableDev& t, int dim, int64_t row, int off) {
  RawChunk r;
  if constexpr (FMT == EG_FMT_Q8_0 || FMT == EG_FMT_MXFP8) {
    const u32x2 q = *(const u32x2*)(t.payload + row * dim + off);
    r.w0 = u32x4{q.x, q.y, 0u, 0u};
    if constexpr (FMT == EG_FMT_Q8_0)
      r.s = *(const uint16_t*)(t.scales + (row * (dim >> 5) + (off >> 5)) * 2);
    else
      r.s = t.scales[row * (dim >> 5) + (off >> 5)];
  } else if constexpr (FMT == EG_FMT_BF16) {
    r.w0 = *(const u32x4*)(t.payload + (row * dim + off) * 2);
  } else if constexpr (FMT == EG_FMT_IQ4_NL) {
    // 18-byte blocks: fp16 d, then 16 bytes of nibbles; value j < 16 is the low
    // nibble of byte j, value j >= 16 the high nibble of byte j-16.  The chunk's
    // 8 nibble bytes start at an even address q: the aligned 8 bytes at q & ~3
    // and the halfword at q + 6 hold them whatever q % 4 is, and no load reaches
    // past the block.
    const uint8_t* blk = t.payload + row * t.stride + (off >> 5) * 18;
    r.s = *(const uint16_t*)blk;
    const uint8_t* q = blk + 2 + (off & 15);
    const uint32_t mis = (uint32_t)(uintptr_t)q & 3u;  // 0 or 2
    const uint32_t* al = (const uint32_t*)(q - mis);  // 4-byte aligned
    const uint32_t d0 = al[0], d1 = al[1];
    const uint32_t tail = *(const uint16_t*)(q + 6);
    r.w0 = u32x4{__builtin_amdgcn_alignbyte(d1, d0, mis), __builtin_amdgcn_alignbyte(tail, d1, mis), 0u, 0u};
  } else {  // EG_FMT_F32
    const u32x4* src = (const u32x4*)(t.payload + (row * dim + off) * 4);
    r.w0 = src[0];
    r.w1 = src[1];
  }
  return r;
}

template <int FMT>
__device__ inline void decode(const RawChunk& r, int off, float v[8]) {
  if constexpr (FMT == EG_FMT_Q8_0) {
    const float d = f16_to_f32((uint16_t)r.s);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)(r.w0[i >> 2] >> ((i & 3) * 8)) * d;
  } else if constexpr (FMT == EG_FMT_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(r.w0[i] << 16);
      v[2 * i + 1] = __uint_as_float(r.w0[i] & 0xffff0000u);
    }
  } else if constexpr (FMT == EG_FMT_MXFP8) {
    const float sc = e8m0_to_f32(r.s);
    e4m3x4_to_f32(r.w0[0], v);
    e4m3x4_to_f32(r.w0[1], v + 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * sc;
  } else if constexpr (FMT == EG_FMT_IQ4_NL) {
    const float d = f16_to_f32((uint16_t)r.s);
    const int sh = ((off & 31) >= 16) ? 4 : 0;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t q = iq4nl_lookup4((r.w0[w] >> sh) & 0x0f0f0f0fu);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * w + i] = (float)(int8_t)(q >> (8 * i)) * d;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = __uint_as_float(r.w0[i]);
      v[4 + i] = __uint_as_float(r.w1[i]);
    }
  }
}

template <int FMT>
__device__ inline void load_chunk(const TableDev& t, int dim, int64_t row, int off, float v[8]) {
  decode<FMT>(load_raw<FMT>(t, dim, row, off), off, v);
}

// Runtime-format variants (overlay rows).
__device__ inline RawChunk load_raw_rt(const TableDev& t, int64_t row, int off) {
  switch (t.fmt) {
    case EG_FMT_Q8_0: return load_raw<EG_FMT_Q8_0>(t, t.dim, row, off);
    case EG_FMT_BF16: return load_raw<EG_FMT_BF16>(t, t.dim, row, off);
    case EG_FMT_MXFP8: return load_raw<EG_FMT_MXFP8>(t, t.dim, row, off);
    case EG_FMT_IQ4_NL: return load_raw<EG_FMT_IQ4_NL>(t, t.dim, row, off);
    default: return load_raw<EG_FMT_F32>(t, t.dim, row, off);
  }
}

__device__ inline void decode_rt(int fmt, const RawChunk& r, int off, float v[8]) {
  switch (fmt) {
    case EG_FMT_Q8_0: decode<EG_FMT_Q8_0>(r, off, v); break;
    case EG_FMT_BF16: decode<EG_FMT_BF16>(r, off, v); break;
    case EG_FMT_MXFP8: decode<EG_FMT_MXFP8>(r, off, v); break;
    case EG_FMT_IQ4_NL: decode<EG_FMT_IQ4_NL>(r, off, v); break;
    default: decode<EG_FMT_F32>(r, off, v); break;
  }
}

__device__ inline void load_chunk_rt(const TableDev& t, int64_t row, int off, float v[8]) {
  decode_rt(t.fmt, load_raw_rt(t, row, off), off, v);
}

// One dequantised value: column `col` of row `row` (any format).
__device__ inline float load_value_rt(const TableDev& t, int64_t row, int col) {
  const int nb = t.dim >> 5;
  switch (t.fmt) {
    case EG_FMT_Q8_0:
      return (float)(int8_t)t.payload[row * t.dim + col] *
             f16_to_f32(((const uint16_t*)t.scales)[row * nb + (col >> 5)]);
    case EG_FMT_BF16:
      return __uint_as_float((uint32_t)((const uint16_t*)t.payload)[row * t.dim + col] << 16);
    case EG_FMT_MXFP8:
      return e4m3_to_f32(t.payload[row * t.dim + col]) * e8m0_to_f32(t.scales[row * nb + (col >> 5)]);
    case EG_FMT_IQ4_NL: {
      const uint8_t* blk = t.payload + row * t.stride + (col >> 5) * 18;
      const int j = col & 31;
      const uint32_t byte = blk[2 + (j & 15)];
      return iq4nl_value(j < 16 ? (byte & 15u) : (byte >> 4)) * f16_to_f32(*(const uint16_t*)blk);
    }
    default:
      return ((const float*)t.payload)[row * t.dim + col];
  }
}

// A 32-bit mix of a row id (xorshift-multiply rounds).
__host__ __device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// The filter block and its five bits of a row in the overlay bitmap's blocked
// Bloom filter (n_fb 64-bit blocks): the block by a multiply-shift of one mix
// of the row, the bits from five 6-bit fields of a second mix.
struct BloomProbe {
  uint32_t block;
  uint64_t mask;
};

__host__ __device__ inline BloomProbe bloom_probe(uint32_t row, uint32_t n_fb) {
  const uint32_t x = mix32(row);
  const uint32_t y = mix32(x ^ 0x9e3779b9u);
  BloomProbe p;
  p.block = (uint32_t)(((uint64_t)x * n_fb) >> 32);
  p.mask = (1ull << (y & 63u)) | (1ull << ((y >> 6) & 63u)) | (1ull << ((y >> 12) & 63u)) |
           (1ull << ((y >> 18) & 63u)) | (1ull << ((y >> 24) & 63u));
  return p;
}

// 32-row words and 64-bit filter blocks of an overlay bitmap over n_bits rows.
__host__ __device__ inline int64_t bitmap_words(int64_t n_bits) { return (n_bits + 31) >> 5; }
__host__ __device__ inline int64_t bitmap_filter_blocks(int64_t n_bits) { return (bitmap_words(n_bits) + 63) >> 6; }

// Index of row in the sorted ids behind an eg_build_id_bitmap rank bitmap, or
// -1.  Layout (nw = ceil(n_bits / 32) words of 32 rows): pairs [2 w] = the
// word's bits, [2 w + 1] = the ids below row 32 w; then ceil(nw / 64) 64-bit
// filter blocks (a blocked Bloom filter of the ids: five bits in one block an
// id).  The filter settles almost every miss from an L2-resident block; a row
// it passes reads its word's pair (bits and rank in one 8-byte load): overlay
// index = rank + popcount of the bits below the row.
__device__ inline int64_t bitmap_find(const uint32_t* __restrict__ bm, int64_t n_bits, int32_t row) {
  const int64_t nw = bitmap_words(n_bits);
  const bool in = (int64_t)(uint32_t)row < n_bits;
  const BloomProbe bp = bloom_probe((uint32_t)row, (uint32_t)bitmap_filter_blocks(n_bits));
  const uint64_t fb = ((const uint64_t*)(bm + 2 * nw))[bp.block];
  int64_t k = -1;
  if (in && (fb & bp.mask) == bp.mask) {
    const uint32_t w = (uint32_t)row >> 5;
    const u32x2 pr = ((const u32x2*)bm)[w];
    const uint32_t bit = (uint32_t)row & 31u;
    if ((pr.x >> bit) & 1u) k = (int64_t)pr.y + __popc(pr.x & ((1u << bit) - 1u));
  }
  return k;
}

__device__ inline int64_t sorted_find(const int32_t* __restrict__ ids, int64_t n, int32_t key) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ids[mid] < key) lo = mid + 1; else hi = mid;
  }
  return (lo < n && ids[lo] == key) ? lo : -1;
}

}  // namespace eg
