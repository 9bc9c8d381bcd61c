// Register-resident pair tiles for the 32x32x16 bf16 MFMA.
//
// A wave holds a tile of 32 pairs x 128 channels as MFMA operands: lane l
// (rho = l & 31, h = l >> 5) owns pair slot rho and the alternate 8-channel
// chunks 2s + h, i.e. for the 8 MFMA k-steps s the lane supplies channels
// 16s + 8h .. 16s + 8h + 7 (a k-permutation of the 128 channels; the weight
// operand reads the same channels, so the product is unchanged).  A pair's two
// lanes thus read adjacent 16-byte chunks: each 16-byte row-load instruction
// covers 32 bytes of one cache line per pair, 32 lines per instruction (64 for
// contiguous half rows, which cost measurably more vector-L1 time).
//
// Pair slots are filled in the order perm32(rho), which makes the
// accumulator of an MFMA whose rows are pair slots come out with every lane
// holding 16 *consecutive* pairs:  D lane (n, h) register u  <->  pair 16h + u.
// The same permutation applied to weight rows makes a lane hold 16
// consecutive output channels.  Both give 32-byte contiguous stores.
#pragma once

#include "common.h"

namespace bioemu {

constexpr int kPairC = 128;          // channels of a pair tile
constexpr int kLdw = kPairC + 8;     // LDS row stride (bf16) of 128-wide weight rows

// rho = 8r + 4h + c  ->  16h + 4r + c
__device__ __forceinline__ int perm32(int rho) {
  return ((rho >> 2) & 1) * 16 + (rho >> 3) * 4 + (rho & 3);
}

// LayerNorm over the 128 channels held by lanes l and l^32 (biased variance,
// two-pass, fp32), gamma/beta fp32 (beta may be null); bf16 result in the
// MFMA operand layout.
__device__ __forceinline__ void layernorm_half_row(const bf16x8 raw[8], const float* __restrict__ gamma,
                                                   const float* __restrict__ beta, int h, float eps,
                                                   bf16x8 out[8]) {
  float v[64];
#pragma unroll
  for (int s = 0; s < 8; ++s) unpack8(raw[s], v + 8 * s);
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 64; ++t) sum += v[t];
  sum += __shfl_xor(sum, 32);
  const float mean = sum * (1.0f / kPairC);
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 64; ++t) {
    const float d = v[t] - mean;
    ss += d * d;
  }
  ss += __shfl_xor(ss, 32);
  const float rstd = rsqrtf(ss * (1.0f / kPairC) + eps);
  // v[8s + e] is channel 16s + 8h + e
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int t = 4 * q, ch = 16 * (t >> 3) + 8 * h + (t & 7);
    const float4 g = *reinterpret_cast<const float4*>(gamma + ch);
    float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
    if (beta) b = *reinterpret_cast<const float4*>(beta + ch);
    out[t >> 3][(t & 7) + 0] = f2bf((v[t + 0] - mean) * rstd * g.x + b.x);
    out[t >> 3][(t & 7) + 1] = f2bf((v[t + 1] - mean) * rstd * g.y + b.y);
    out[t >> 3][(t & 7) + 2] = f2bf((v[t + 2] - mean) * rstd * g.z + b.z);
    out[t >> 3][(t & 7) + 3] = f2bf((v[t + 3] - mean) * rstd * g.w + b.w);
  }
}

// Channel-major projection block: 32 pair slots x 32 output channels.
//   acc = X(32 x 128) * W[row0 .. row0+31, :]^T       (W in LDS, stride kLdw)
// D lane (n, h): output channel row0 + n, register u <-> pair slot 16h + u.
__device__ __forceinline__ f32x16 proj_block_cm(const bf16x8 x[8], const bf16* wl, int row0, int n,
                                                int h) {
  f32x16 acc = zero16();
  const bf16* w = wl + (row0 + n) * kLdw + 8 * h;
#pragma unroll
  for (int s = 0; s < 8; ++s) acc = mfma32(x[s], load8(w + 16 * s), acc);
  return acc;
}

// Pair-major projection block: 32 output channels x 32 pair slots.
//   acc = W[row0 + perm32(.), :] * X^T
// D lane (n, h): pair slot perm32(n), register u <-> output channel row0 + 16h + u.
__device__ __forceinline__ f32x16 proj_block_pm(const bf16x8 x[8], const bf16* wl, int row0, int n,
                                                int h) {
  f32x16 acc = zero16();
  const bf16* w = wl + (row0 + perm32(n)) * kLdw + 8 * h;
#pragma unroll
  for (int s = 0; s < 8; ++s) acc = mfma32(load8(w + 16 * s), x[s], acc);
  return acc;
}

// ---------------------------------------------------------------------------
// LayerNorm folded into the projection that follows it.
//
//   LN(x) W^T = xhat (W diag(gamma))^T + W beta,   xhat = (x - mean) * rstd
//
// launch_fold_ln (fold.hip) writes W' = W diag(gamma) (bf16, [rows][128]) and the bias
// W beta split into two bf16 parts (hi + lo, ~16 mantissa bits together,
// [rows][2]).  Kernels normalise affine-free (no gamma/beta registers) and
// add the bias with one extra MFMA k-step: x-side operand [keep, keep, 0..]
// against weight-side [hi, lo, 0..].  keep = 0 zeroes a pair's whole output
// (its xhat row is zeroed too), which is the masked_fill of the reference
// for bias-free projections.
// ---------------------------------------------------------------------------
// Affine-free LayerNorm of the 128 channels held by lanes l and l^32 (this
// lane's 64 in v, fp32), bf16 result in the MFMA operand layout; a row with
// keep == false comes out zero.
__device__ __forceinline__ void normalize_half_row(const float* v, bool keep, bf16x8 out[8]) {
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < 64; ++c) sum += v[c];
  sum += __shfl_xor(sum, 32);
  const float mean = sum * (1.0f / kPairC);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < 64; ++c) {
    const float d = v[c] - mean;
    ss += d * d;
  }
  ss += __shfl_xor(ss, 32);
  const float rstd = keep ? rsqrtf(ss * (1.0f / kPairC) + 1e-5f) : 0.f;
#pragma unroll
  for (int c = 0; c < 64; ++c) out[c >> 3][c & 7] = f2bf((v[c] - mean) * rstd);
}

// Loads this lane's 64 channels of a pair row (chunks 2s + h) as fp32 (zeros
// when !valid).
__device__ __forceinline__ void load_half_row_f32(const bf16* row, int h, bool valid, float* v) {
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    bf16x8 raw;
    if (valid) {
      raw = load8(row + 8 * h + 16 * s);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) raw[t] = f2bf(0.f);
    }
    unpack8(raw, v + 8 * s);
  }
}

// x-side operand of the bias k-step: [keep, keep, 0, ...] in the lanes h = 0 (k slots 0 and 1).
__device__ __forceinline__ bf16x8 bias_step_x(bool keep, int h) {
  bf16x8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = f2bf(0.f);
  if (h == 0 && keep) {
    r[0] = f2bf(1.f);
    r[1] = f2bf(1.f);
  }
  return r;
}

// weight-side operand of the bias k-step for weight row `row`: [hi, lo, 0, ...].
__device__ __forceinline__ bf16x8 bias_step_w(const bf16* cl, int row, int h) {
  bf16x8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = f2bf(0.f);
  if (h == 0) {
    r[0] = cl[2 * row];
    r[1] = cl[2 * row + 1];
  }
  return r;
}

// Channel-major folded projection block: X(32 x 128) W'[row0..+31]^T + keep * c.
__device__ __forceinline__ f32x16 proj_block_cm_f(const bf16x8 x[8], bf16x8 xb, const bf16* wl, const bf16* cl,
                                                  int row0, int n, int h) {
  f32x16 acc = zero16();
  const bf16* w = wl + (row0 + n) * kLdw + 8 * h;
#pragma unroll
  for (int s = 0; s < 8; ++s) acc = mfma32(x[s], load8(w + 16 * s), acc);
  return mfma32(xb, bias_step_w(cl, row0 + n, h), acc);
}

// Pair-major folded projection block: W'[row0 + perm32(.)] X^T + c * keep.
__device__ __forceinline__ f32x16 proj_block_pm_f(const bf16x8 x[8], bf16x8 xb, const bf16* wl, const bf16* cl,
                                                  int row0, int n, int h) {
  f32x16 acc = zero16();
  const int r = row0 + perm32(n);
  const bf16* w = wl + r * kLdw + 8 * h;
#pragma unroll
  for (int s = 0; s < 8; ++s) acc = mfma32(load8(w + 16 * s), x[s], acc);
  return mfma32(bias_step_w(cl, r, h), xb, acc);
}

// Copies `rows` bias pairs (hi, lo) into LDS, zero-filling up to rows_padded.
__device__ __forceinline__ void stage_bias(bf16* cl, const bf16* __restrict__ cf, int rows, int rows_padded) {
  for (int q = threadIdx.x; q < 2 * rows_padded; q += blockDim.x) cl[q] = q < 2 * rows ? cf[q] : f2bf(0.f);
}

// 16 fp32 accumulator values -> two 16-byte bf16 chunks.
__device__ __forceinline__ void store16(bf16* dst, const float* v) {
  bf16x8 a, b;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    a[t] = f2bf(v[t]);
    b[t] = f2bf(v[8 + t]);
  }
  store8(dst, a);
  store8(dst + 8, b);
}

// Copies `rows` x 128 bf16 weight rows from global memory into LDS (stride
// kLdw) and zero-fills rows [rows, rows_padded).  Whole workgroup; no barrier.
__device__ __forceinline__ void stage_weights(bf16* wl, const bf16* __restrict__ w, int rows,
                                              int rows_padded) {
  const int chunks = rows_padded * (kPairC / 8);
  for (int q = threadIdx.x; q < chunks; q += blockDim.x) {
    const int r = q >> 4, part = q & 15;
    bf16x8 v;
    if (r < rows) {
      v = load8(w + (size_t)r * kPairC + part * 8);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = f2bf(0.f);
    }
    store8(wl + r * kLdw + part * 8, v);
  }
}

}  // namespace bioemu
