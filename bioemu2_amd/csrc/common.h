// Shared device helpers for the gfx950 (MI355X, CDNA4) Pairformer kernels.
//
// Conventions used by every kernel in this library:
//   * Activations in HBM are bf16, channel-last ([B, N, N, C] for pair tensors).
//   * Arithmetic: bf16 MFMA operands with fp32 accumulation; LayerNorm
//     statistics, softmax and gating in fp32 registers.
//   * Wavefront = 64 lanes; workgroups are 4 to 16 waves.
//
// MFMA 32x32x16 bf16 (v_mfma_f32_32x32x16_bf16), D[32x32] += A[32x16] * B[16x32].
// Lane l (0..63), h = l >> 5, n = l & 31:
//   A operand: 8 bf16, row n, k = 8h .. 8h+7
//   B operand: 8 bf16, col n, k = 8h .. 8h+7
//   D (16 fp32): col n, reg 4r+c holds row 8r + 4h + c   (r, c in 0..3)
// The k index inside one MFMA may be permuted freely as long as A and B use
// the same permutation; kernels that feed an accumulator back in as the next
// B operand use  kappa(h, t) = (t < 4) ? 4h + t : 8 + 4h + (t - 4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bioemu {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ float bf2f(bf16 v) { return (float)v; }
__device__ __forceinline__ bf16 f2bf(float v) { return (bf16)v; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// sigmoid(x) = 1 / (1 + exp(-x)); exp overflow gives rcp(inf) = 0 as required.
__device__ __forceinline__ float sigmoidf_fast(float x) {
  return fast_rcp(1.0f + fast_exp2(-x * kLog2e));
}

// silu(x) = x * sigmoid(x)
__device__ __forceinline__ float siluf_fast(float x) { return x * sigmoidf_fast(x); }

__device__ __forceinline__ bf16x8 load8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ void store8(bf16* p, bf16x8 v) { *reinterpret_cast<bf16x8*>(p) = v; }

// This thread's wave within the workgroup as a wave-uniform (scalar) value.
// Everything derived from it (tile indices, base pointers, buffer resources)
// then stays in scalar registers; derived from plain threadIdx.x the compiler
// must treat it as per-lane, and every buffer load through a resource built
// from it becomes a readfirstlane loop.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Flat tile index t = (b * rows + row) * cols + col -> (b, row, col) in 32-bit
// arithmetic (launchers keep tile counts below 2^31).
struct TileIdx {
  int b, row, col;
};
__device__ __forceinline__ TileIdx split_tile(unsigned t, unsigned cols, unsigned rows) {
  const unsigned r = t / cols, b = r / rows;
  return {(int)b, (int)(r - b * rows), (int)(t - r * cols)};
}

// Buffer resource over [base, base + bytes) (raw buffer, 32-bit offsets).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16-byte load at byte offset voff (per lane) + soff (wave-uniform).
__device__ __forceinline__ bf16x8 buffer_load8(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return __builtin_bit_cast(bf16x8, v);
}

// acc + sum of the eight bf16 values of v (four bf16 dot2 steps against ones).
__device__ __forceinline__ float sum8_bf16(bf16x8 v, float acc) {
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const bf16x2 pair = {v[2 * t], v[2 * t + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(pair, one, acc, false);
  }
  return acc;
}

// A 16-byte chunk as eight bf16 -> fp32 values.
__device__ __forceinline__ void unpack8(bf16x8 v, float* out) {
#pragma unroll
  for (int t = 0; t < 8; ++t) out[t] = bf2f(v[t]);
}

// ---------------------------------------------------------------------------
// Residual tails.  A residual stream (the pair tensor z, the single s, the
// MSA m) can be carried at ~16 significant bits as its bf16 value hi plus one
// int8 "tail" t per element:
//   value = hi + t * 2^(E - 142),   E = biased exponent field of hi,
// so t counts 1/256ths of hi's unit in the last place (ulp = 2^(E - 134) for
// a normal hi).  hi is the round-to-nearest bf16 of the value, so the
// remainder is at most half an ulp (|t| <= 128, clamped to 127).  Kernels that
// only *read* the stream (LayerNorm inputs) use hi; kernels that add a
// residual read hi + tail and write the sum back as a new (hi, tail).  Tail
// planes have the layout of their stream with one byte per element.
// ---------------------------------------------------------------------------
// The helpers work on the fp32 bit pattern of hi (a bf16 widened to fp32 is
// its 16 bits shifted up), so the exponent field is one bit-field extract of a
// 32-bit register.
__device__ __forceinline__ int f32_exp_field(uint32_t bits) { return (int)((bits >> 23) & 0xffu); }

// hi + t * 2^(E(hi) - 142), hi given as its fp32 bit pattern
__device__ __forceinline__ float tail_decode_bits(uint32_t hb, int t) {
  return __builtin_bit_cast(float, hb) + __builtin_amdgcn_ldexpf((float)t, f32_exp_field(hb) - 142);
}

// Sixteen consecutive elements: raw bf16 halves r0, r1 and their 16 tail bytes
// -> fp32 values.
__device__ __forceinline__ void tail_decode16(bf16x8 r0, bf16x8 r1, u32x4 tb, float* v) {
  const u32x4 w0 = __builtin_bit_cast(u32x4, r0), w1 = __builtin_bit_cast(u32x4, r1);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const uint32_t w = u < 8 ? w0[(u >> 1) & 3] : w1[(u >> 1) & 3];
    const uint32_t hb = (u & 1) ? (w & 0xffff0000u) : (w << 16);
    const int t = __builtin_amdgcn_sbfe((int)tb[u >> 2], 8 * (u & 3), 8);
    v[u] = tail_decode_bits(hb, t);
  }
}

// Sixteen fp32 values -> bf16 halves a (values 0-7), b (8-15) and their tail bytes.
// t = clamp(round(r * 2^(142 - E)), -127, 127) with r = v - hi exact: the
// remainder is clamped first and rounded to nearest even by adding 1.5 * 2^23,
// which leaves t in the low byte of the sum's bit pattern (two's complement);
// clamping before or after rounding gives the same integer.
__device__ __forceinline__ void tail_encode16(const float* v, bf16x8& a, bf16x8& b, u32x4& tb) {
  uint32_t y[16];
#pragma unroll
  for (int u = 0; u < 16; u += 2) {
    const bf16x2 hp = {f2bf(v[u]), f2bf(v[u + 1])};
    const uint32_t w = __builtin_bit_cast(uint32_t, hp);
    if (u < 8) {
      a[u] = hp[0];
      a[u + 1] = hp[1];
    } else {
      b[u - 8] = hp[0];
      b[u - 7] = hp[1];
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t hb = e ? (w & 0xffff0000u) : (w << 16);
      const float r = __builtin_amdgcn_ldexpf(v[u + e] - __builtin_bit_cast(float, hb), 142 - f32_exp_field(hb));
      y[u + e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_fmed3f(r, -127.f, 127.f) + 12582912.0f);
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    // low bytes of y[4k .. 4k + 3] -> bytes 0..3 of word k
    const uint32_t lo = __builtin_amdgcn_perm(y[4 * k + 1], y[4 * k], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(y[4 * k + 3], y[4 * k + 2], 0x0c0c0400u);
    tb[k] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  }
}

// Sixteen fp32 values -> bf16 halves (stored at dst, dst + 8) and tail bytes.
__device__ __forceinline__ void tail_store16(bf16* dst, int8_t* tdst, const float* v) {
  bf16x8 a, b;
  u32x4 tb;
  tail_encode16(v, a, b, tb);
  *reinterpret_cast<bf16x8*>(dst) = a;
  *reinterpret_cast<bf16x8*>(dst + 8) = b;
  *reinterpret_cast<u32x4*>(tdst) = tb;
}

__device__ __forceinline__ u32x4 load_tail16(const int8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Pair-interleaved channel layout (the two lanes l and l ^ 32 of a pair slot
// hold alternate 8-channel chunks, lane h chunk s = channels 16 s + 8 h + 0..7):
// tail words of 16 channels exchanged between the two lanes.  Lane h = 0 keeps
// words 0-1 and takes the partner's 0-1 as 2-3; lane h = 1 takes the
// partner's 2-3 as 0-1 and keeps 2-3.  The same exchange turns loaded bytes
// (contiguous channels 32 cb + 16 h + 0..15) into the lane's interleaved
// order (32 cb + 8 h + 0..7, then 32 cb + 16 + 8 h + 0..7) and the lane's
// encoded bytes back into contiguous ones.  Both lanes must be active.
__device__ __forceinline__ u32x4 exchange_tail_halves(u32x4 d, int h) {
  const int s0 = (int)(h ? d[0] : d[2]), s1 = (int)(h ? d[1] : d[3]);
  const unsigned r0 = (unsigned)__shfl_xor(s0, 32), r1 = (unsigned)__shfl_xor(s1, 32);
  u32x4 o;
  o[0] = h ? r0 : d[0];
  o[1] = h ? r1 : d[1];
  o[2] = h ? d[2] : r0;
  o[3] = h ? d[3] : r1;
  return o;
}

}  // namespace bioemu
