// fp32 arithmetic path of the denoiser's ops, for gfx950.
//
// The reference runs its denoiser with autocast off (src/bioemu2/biomoa/models/
// score_model.py:355, model.py:387), so its attention-with-pair-bias
// (attention_pair_bias.py:128-225), sliding-window attention (:277-340) and
// token transitions (transition.py:52-91) compute in fp32 on fp32 inputs.  These
// entry points do the same: fp32 operands and fp32 accumulation throughout.
//
//   gemm_f32      out = epi(A W^T) on v_mfma_f32_32x32x2_f32 (qkvg_f32: the four
//                 token projections of an attention in one launch).  A wave owns a
//                 32 x 32 output block: weight rows (output channels) are the
//                 MFMA A operand in perm32 order (pairtile.h), token rows the B
//                 operand, so a lane ends with 16 consecutive channels of one
//                 row (64-byte stores).  Each lane loads 4 consecutive k of its
//                 row per step (16 bytes) and feeds them to 4 MFMAs: lane half h
//                 supplies k0 + 4h + e to MFMA e, the same k permutation on both
//                 operands, so every k is summed once.
//   rows_ln_f32   LayerNorm per row (biased variance, eps 1e-5), one wave per row.
//   pair_proj_f32 pair bias: LN(z) W^T per pair row, one thread per row, written
//                 head-major ([outer][head][inner]).
//   attn_f32      softmax(q k^T / sqrt(d) + bias; masked keys -> -1e6) v, gated by
//                 g: flash attention on the same fp32 MFMA, a wave per 32
//                 queries, 32-key blocks, online softmax in registers.
//   swa_attn_f32  the same over the sliding key window of each 32-atom window.
#include <algorithm>
#include <cmath>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmEpiStore = 0, kGemmEpiSigmoid = 1, kGemmEpiSwiGLU = 2, kGemmEpiResidual = 3;
// kGemmEpiStoreT writes the transpose per sequence: row m = s * T + t, channel
// c -> out[(s * N + c) * ldT + t] (keys contiguous, for the P.V operand).
constexpr int kGemmEpiStoreT = 4;

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int kEpi>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ W,
                                                       const float* __restrict__ W2, const float* __restrict__ bias,
                                                       const float* res, float* out, long long M, int K, int N,
                                                       int T, int ldT) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int nbc = N / 32;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  const long long mblocks = (M + 31) / 32;
  if (blk >= mblocks * nbc) return;   // no barriers in this kernel
  const long long mb = blk / nbc;
  const int cb = (int)(blk % nbc);
  const long long m = mb * 32 + n;
  const bool mvalid = m < M;
  const float* arow = A + (size_t)(mvalid ? m : 0) * K + 4 * h;
  const size_t wr = (size_t)(cb * 32 + perm32(n)) * K + 4 * h;
  const float* wrow = W + wr;
  const float* w2row = kEpi == kGemmEpiSwiGLU ? W2 + wr : nullptr;
  f32x16 acc = zero16(), acc2 = zero16();
  for (int k0 = 0; k0 < K; k0 += 8) {
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(arow + k0);
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(wrow + k0);
    f32x4 v4;
    if (kEpi == kGemmEpiSwiGLU) v4 = *reinterpret_cast<const f32x4*>(w2row + k0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = mfma_f32(w4[e], a4[e], acc);
      if (kEpi == kGemmEpiSwiGLU) acc2 = mfma_f32(v4[e], a4[e], acc2);
    }
  }
  if (!mvalid) return;
  // D lane (n, h): token row m, register u <-> output channel cb*32 + 16h + u
  const int c0 = cb * 32 + 16 * h;
  float v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    float x = acc[u];
    if (bias) x += bias[c0 + u];
    if (kEpi == kGemmEpiSigmoid) x = 1.0f / (1.0f + __expf(-x));
    if (kEpi == kGemmEpiSwiGLU) x = x / (1.0f + __expf(-x)) * acc2[u];
    v[u] = x;
  }
  if (kEpi == kGemmEpiStoreT) {
    const long long sq = m / T, t = m % T;
    float* col = out + ((size_t)sq * N + c0) * ldT + t;
#pragma unroll
    for (int u = 0; u < 16; ++u) col[(size_t)u * ldT] = v[u];
    return;
  }
  float* dst = out + (size_t)m * N + c0;
  if (kEpi == kGemmEpiResidual) {
    const float* r = res + (size_t)m * N + c0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 rv = *reinterpret_cast<const f32x4*>(r + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * q + e] += rv[e];
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 o4;
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = v[4 * q + e];
    *reinterpret_cast<f32x4*>(dst + 4 * q) = o4;
  }
}

// The four token projections of an attention in one launch: column blocks
// [0, c_s) -> q (+ q bias), [c_s, 2c_s) -> k, [2c_s, 3c_s) -> v stored
// transposed per sequence (as kGemmEpiStoreT), [3c_s, 4c_s) -> sigmoid(g).
// Same wave tiling as gemm_f32_kernel; the column block picks weight rows and
// epilogue (wave-uniform).
__global__ __launch_bounds__(256) void qkvg_f32_kernel(const float* __restrict__ A, const float* __restrict__ w_qkv,
                                                       const float* __restrict__ w_g, const float* __restrict__ q_bias,
                                                       float* __restrict__ q, float* __restrict__ k,
                                                       float* __restrict__ vt, float* __restrict__ g, long long M,
                                                       int c_s, int T, int ldT) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int nbc = c_s / 32;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  const long long mblocks = (M + 31) / 32;
  if (blk >= mblocks * 4 * nbc) return;   // no barriers in this kernel
  const long long mb = blk / (4 * nbc);
  const int cbt = (int)(blk % (4 * nbc));
  const int part = cbt / nbc, cb = cbt % nbc;
  const long long m = mb * 32 + n;
  const bool mvalid = m < M;
  const int K = c_s;
  const float* arow = A + (size_t)(mvalid ? m : 0) * K + 4 * h;
  const float* wbase = part < 3 ? w_qkv + (size_t)part * c_s * c_s : w_g;
  const float* wrow = wbase + (size_t)(cb * 32 + perm32(n)) * K + 4 * h;
  f32x16 acc = zero16();
  for (int k0 = 0; k0 < K; k0 += 8) {
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(arow + k0);
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(wrow + k0);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = mfma_f32(w4[e], a4[e], acc);
  }
  if (!mvalid) return;
  const int c0 = cb * 32 + 16 * h;
  if (part == 2) {
    const long long sq = m / T, t = m % T;
    float* col = vt + ((size_t)sq * c_s + c0) * ldT + t;
#pragma unroll
    for (int u = 0; u < 16; ++u) col[(size_t)u * ldT] = acc[u];
    return;
  }
  float v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    float x = acc[u];
    if (part == 0 && q_bias) x += q_bias[c0 + u];
    if (part == 3) x = 1.0f / (1.0f + __expf(-x));
    v[u] = x;
  }
  float* dst = (part == 0 ? q : part == 1 ? k : g) + (size_t)m * c_s + c0;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    f32x4 o4;
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = v[4 * qd + e];
    *reinterpret_cast<f32x4*>(dst + 4 * qd) = o4;
  }
}

// LayerNorm of the row [x1 row (K1 values) | x2 row (K2 values)], the concatenation read in place.
__global__ __launch_bounds__(256) void rows_ln_f32_kernel(const float* __restrict__ x1, int K1,
                                                          const float* __restrict__ x2, int K2,
                                                          const float* __restrict__ g, const float* __restrict__ b,
                                                          float* __restrict__ y, long long rows) {
  const int lane = threadIdx.x & 63;
  const long long r = (long long)blockIdx.x * 4 + wave_id();
  if (r >= rows) return;
  const int K = K1 + K2;
  const float* r1 = x1 + (size_t)r * K1;
  const float* r2 = x2 + (size_t)r * K2;   // read only when K2 > 0
  auto at = [&](int k) { return k < K1 ? r1[k] : r2[k - K1]; };
  float s = 0.f;
  for (int k = lane; k < K; k += 64) s += at(k);
  const float mean = wave_sum(s) / (float)K;
  float ss = 0.f;
  for (int k = lane; k < K; k += 64) {
    const float d = at(k) - mean;
    ss += d * d;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)K + 1e-5f);
  float* yr = y + (size_t)r * K;
  for (int k = lane; k < K; k += 64) yr[k] = (at(k) - mean) * rstd * g[k] + (b ? b[k] : 0.f);
}

// Pair bias LN(z) W^T, one thread per pair row: every lane reads the same
// weight, so the head loop's weight reads are wave-uniform.
template <int CZ>
__global__ __launch_bounds__(256) void pair_proj_f32_kernel(const float* __restrict__ z, const float* __restrict__ g,
                                                            const float* __restrict__ b, const float* __restrict__ w,
                                                            float* __restrict__ out, long long P, int nrows, int ncols,
                                                            int ld, int H) {
  const long long p = (long long)blockIdx.x * 256 + threadIdx.x;
  if (p >= P) return;
  float v[CZ];
  const f32x4* src = reinterpret_cast<const f32x4*>(z + (size_t)p * CZ);
#pragma unroll
  for (int q = 0; q < CZ / 4; ++q) {
    const f32x4 t = src[q];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CZ; ++c) s += v[c];
  const float mean = s / (float)CZ;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CZ; ++c) {
    const float d = v[c] - mean;
    ss += d * d;
  }
  const float rstd = 1.0f / sqrtf(ss / (float)CZ + 1e-5f);
#pragma unroll
  for (int c = 0; c < CZ; ++c) v[c] = (v[c] - mean) * rstd * g[c] + (b ? b[c] : 0.f);
  const long long inner = (long long)nrows * ncols;
  const long long outer = p / inner, idx = p % inner;
  const long long r = idx / ncols, col = idx % ncols;
  for (int hh = 0; hh < H; ++hh) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CZ; ++c) acc += w[hh * CZ + c] * v[c];
    out[(((size_t)outer * H + hh) * nrows + r) * ld + col] = acc;
  }
}

// ---------------------------------------------------------------------------
// Flash attention on fp32 MFMA.  A wave owns 32 queries of one (copy, head)
// and walks 32-key blocks:
//   S^T = K Q^T       d/2 MFMAs; lane (r, h) supplies key row r, d-slots
//                     h*d/2 + e (A) and query r's same d-slots (B), so lane
//                     (n, h) ends with query n's logits for keys
//                     8*(u/4) + 4h + u%4 (register u);
//   softmax           blockwise online softmax in registers (max over the
//                     lane pair n, n+32 by one shuffle);
//   O^T = V^T P^T     16 MFMAs of 2 keys: MFMA e takes register e of P (key
//                     8*(e/4) + 4h + e%4 in lane half h) and, as A, V^T at
//                     channel c = lane % 32 (zero for c >= d) and that key.
// Lane (n, h) ends with channels 8*(u/4) + 4h + u%4 of query n.
// Logits follow the reference: q.k / sqrt(d) + bias, a masked key's logit
// replaced by -1e6; keys past the sequence are left out (weight 0).
// ---------------------------------------------------------------------------
template <int D>
struct F32KeyBlock {
  f32x4 k[D / 8];     // K row (key k0 + n), d-slots h*d/2 ..
  f32x4 bias[4];      // bias of query n at keys k0 + 8j + 4h + 0..3
  f32x4 v[4];         // V^T at channel n, keys k0 + 8j + 4h + 0..3
  unsigned keep;      // bit u: key of register u unmasked
  unsigned live;      // bit u: key of register u exists (else weight 0)
};

// Mask bytes of keys 8j + 4h + 0..3 (one 32-bit word per j) -> keep bits.
__device__ __forceinline__ unsigned keep_bits(const unsigned (&w)[4]) {
  unsigned keep = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t) keep |= (unsigned)(((w[j] >> (8 * t)) & 0xffu) != 0u) << (4 * j + t);
  return keep;
}

template <int D>
__device__ __forceinline__ void f32_attend_block(const F32KeyBlock<D>& kb, const float (&qv)[D / 2], float rsq,
                                                 f32x16& o, float& m, float& l) {
  f32x16 s = zero16();
#pragma unroll
  for (int e = 0; e < D / 2; ++e) s = mfma_f32(kb.k[e >> 2][e & 3], qv[e], s);
  float x[16];
  float bmax = -INFINITY;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const float logit = ((kb.keep >> u) & 1u) ? s[u] * rsq + kb.bias[u >> 2][u & 3] : -1e6f;
    x[u] = ((kb.live >> u) & 1u) ? logit : -INFINITY;
    bmax = fmaxf(bmax, x[u]);
  }
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
  const float m_new = fmaxf(m, bmax);
  const float alpha = __expf(m - m_new);
  l *= alpha;
#pragma unroll
  for (int u = 0; u < 16; ++u) o[u] *= alpha;
  float p[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    p[u] = __expf(x[u] - m_new);
    l += p[u];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) o = mfma_f32(kb.v[e >> 2][e & 3], p[e], o);
  m = m_new;
}

// Writes g * o / l for this lane's channels (lane (n, h): 8j + 4h + 0..3).
template <int D>
__device__ __forceinline__ void f32_attend_store(const f32x16& o, float l, const float* g, float* go, bool store) {
  l += __shfl_xor(l, 32);
  if (!store) return;
  const float inv = 1.0f / l;
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = 8 * j + 4 * h;
    if (c < D) {
      const f32x4 gv = *reinterpret_cast<const f32x4*>(g + c);
      f32x4 r;
#pragma unroll
      for (int t = 0; t < 4; ++t) r[t] = gv[t] * (o[4 * j + t] * inv);
      *reinterpret_cast<f32x4*>(go + c) = r;
    }
  }
}

template <int D>
__device__ __forceinline__ void load_q_f32(const float* qr, float (&qv)[D / 2]) {
#pragma unroll
  for (int j = 0; j < D / 8; ++j) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(qr + 4 * j);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[4 * j + e] = t[e];
  }
}

// Full attention: grid (ceil(N / 128), H, B * mult), 4 waves of 32 queries
// sharing each 32-key block of K, V^T and the mask through LDS (staged once
// per workgroup, double-buffered).  bias [B][H][N][ld], V^T [B*mult][c_s][ld]
// (ld = N rounded up to 32; columns >= N unused).  Key mask: one row of N
// bytes per batch ([B][N], mask_per_copy = 0) or per copy ([B*mult][N],
// mask_per_copy = 1: triangle attention's per-sequence mask).
template <int D>
__global__ __launch_bounds__(256) void attn_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ vt, const float* __restrict__ g,
                                                       const float* __restrict__ bias,
                                                       const uint8_t* __restrict__ mask, float* __restrict__ go,
                                                       int N, int ld, int H, int c_s, int mult, float rsq,
                                                       int mask_per_copy) {
  constexpr int KS = D + 4, VS = 36, KQ = D / 4;
  __shared__ __attribute__((aligned(16))) float ks[2][32][KS];
  __shared__ __attribute__((aligned(16))) float vs[2][D][VS];
  __shared__ __attribute__((aligned(16))) uint8_t ms[2][32];
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int hd = blockIdx.y, bm = blockIdx.z, b = bm / mult;
  const int q0 = (blockIdx.x * 4 + wave_id()) * 32;
  // waves past N run on a clamped row and store nothing: they stage their
  // share of every block and meet every barrier
  const int qi = min(q0 + n, N - 1);
  float qv[D / 2];
  load_q_f32<D>(q + ((size_t)bm * N + qi) * c_s + hd * D + h * (D / 2), qv);
  const float* brow = bias + (((size_t)b * H + hd) * N + qi) * ld;
  const float* kbase = k + (size_t)bm * N * c_s + hd * D;
  const float* vtb = vt + ((size_t)bm * c_s + hd * D) * ld;
  const uint8_t* mrow = mask + (size_t)(mask_per_copy ? bm : b) * N;
  // staging: thread tid moves K float4 (key tid / KQ, chunk tid % KQ) and
  // V^T float4 (channel tid / 8, keys 4 (tid % 8) ..), thread tid < 32 a mask byte
  const int sk_key = tid / KQ, sk_chunk = tid % KQ;
  const int sv_row = tid >> 3, sv_chunk = tid & 7;
  f32x4 rk, rv;
  uint8_t rm = 0;
  auto gload = [&](int k0) {
    if (tid < 32 * KQ) rk = *reinterpret_cast<const f32x4*>(kbase + (size_t)min(k0 + sk_key, N - 1) * c_s + 4 * sk_chunk);
    if (tid < D * 8) {
      rv = *reinterpret_cast<const f32x4*>(vtb + (size_t)sv_row * ld + k0 + 4 * sv_chunk);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (k0 + 4 * sv_chunk + e >= N) rv[e] = 0.f;   // unwritten columns past N
    }
    if (tid < 32) rm = k0 + tid < N ? mrow[k0 + tid] : 0;
  };
  auto lstore = [&](int st) {
    if (tid < 32 * KQ) *reinterpret_cast<f32x4*>(&ks[st][sk_key][4 * sk_chunk]) = rk;
    if (tid < D * 8) *reinterpret_cast<f32x4*>(&vs[st][sv_row][4 * sv_chunk]) = rv;
    if (tid < 32) ms[st][tid] = rm;
  };
  auto bload = [&](int k0, f32x4 (&bb)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bb[j] = *reinterpret_cast<const f32x4*>(brow + k0 + 8 * j + 4 * h);
  };
  f32x16 o = zero16();
  float m = -INFINITY, l = 0.f;
  F32KeyBlock<D> kb;
  f32x4 bnext[4];
  gload(0);
  bload(0, kb.bias);
  lstore(0);
  __syncthreads();
  int st = 0;
#pragma unroll 1
  for (int k0 = 0; k0 < N; k0 += 32) {
    const bool more = k0 + 32 < N;
    if (more) {
      gload(k0 + 32);
      bload(k0 + 32, bnext);
    }
#pragma unroll
    for (int j = 0; j < D / 8; ++j) kb.k[j] = *reinterpret_cast<const f32x4*>(&ks[st][n][h * (D / 2) + 4 * j]);
    unsigned w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kb.v[j] = n < D ? *reinterpret_cast<const f32x4*>(&vs[st][n < D ? n : 0][8 * j + 4 * h]) : f32x4{0.f, 0.f, 0.f, 0.f};
      w[j] = *reinterpret_cast<const unsigned*>(&ms[st][8 * j + 4 * h]);
    }
    kb.keep = keep_bits(w);
    kb.live = 0u;
#pragma unroll
    for (int u = 0; u < 16; ++u) kb.live |= (unsigned)(k0 + 8 * (u >> 2) + 4 * h + (u & 3) < N) << u;
    f32_attend_block<D>(kb, qv, rsq, o, m, l);
    if (more) {
      lstore(st ^ 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) kb.bias[j] = bnext[j];
    }
    __syncthreads();
    st ^= 1;
  }
  const size_t off = ((size_t)bm * N + qi) * c_s + hd * D;
  f32_attend_store<D>(o, l, g + off, go + off, q0 + n < N);
}

// Sliding-window attention: grid (NW, ceil(heads / 4), B * mult); wave = head,
// its 32 queries are window w's atoms, its keys the Hk positions starting
// (Hk - 32) / 2 before the window (outside the sequence: masked, v = 0; a
// group of 4 keys 4-aligned is wholly inside or outside).  bias
// [B * NW][heads][32][Hk], V^T [B*mult][c_s][NA].
__global__ __launch_bounds__(256) void swa_attn_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ vt, const float* __restrict__ g,
                                                           const float* __restrict__ bias,
                                                           const uint8_t* __restrict__ mask, float* __restrict__ go,
                                                           int NW, int Hk, int heads, int c_s, int mult, float rsq) {
  constexpr int D = 32, W = 32;
  const int lane = threadIdx.x & 63, n = lane & 31, h = lane >> 5;
  const int w = blockIdx.x, bm = blockIdx.z, b = bm / mult;
  const int hd = blockIdx.y * 4 + wave_id();
  if (hd >= heads) return;   // no barriers in this kernel
  const int NA = NW * W, ctx = (Hk - W) / 2;
  const int aq = w * W + n;
  float qv[D / 2];
  load_q_f32<D>(q + ((size_t)bm * NA + aq) * c_s + hd * D + h * (D / 2), qv);
  const float* brow = bias + ((((size_t)b * NW + w) * heads + hd) * W + n) * Hk;
  const float* kbase = k + (size_t)bm * NA * c_s + hd * D;
  const float* vtrow = vt + ((size_t)bm * c_s + hd * D + n) * NA;
  const uint8_t* mrow = mask + (size_t)b * NA;
  const int a0 = w * W - ctx;
  auto fetch = [&](int t0, F32KeyBlock<D>& kb) {
    const float* kr = kbase + (size_t)min(max(a0 + t0 + n, 0), NA - 1) * c_s + h * (D / 2);
#pragma unroll
    for (int j = 0; j < D / 8; ++j) kb.k[j] = *reinterpret_cast<const f32x4*>(kr + 4 * j);
    unsigned mw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kb.bias[j] = *reinterpret_cast<const f32x4*>(brow + t0 + 8 * j + 4 * h);
      const int a = a0 + t0 + 8 * j + 4 * h;
      const bool in = a >= 0 && a < NA;
      kb.v[j] = in ? *reinterpret_cast<const f32x4*>(vtrow + a) : f32x4{0.f, 0.f, 0.f, 0.f};
      mw[j] = in ? *reinterpret_cast<const unsigned*>(mrow + a) : 0u;
    }
    kb.keep = keep_bits(mw);
    kb.live = 0xffffu;
  };
  f32x16 o = zero16();
  float m = -INFINITY, l = 0.f;
  F32KeyBlock<D> cur, nxt;
  fetch(0, cur);
#pragma unroll 1
  for (int t0 = 0; t0 < Hk; t0 += 32) {
    if (t0 + 32 < Hk) fetch(t0 + 32, nxt);
    f32_attend_block<D>(cur, qv, rsq, o, m, l);
    cur = nxt;
  }
  const size_t off = ((size_t)bm * NA + aq) * c_s + hd * D;
  f32_attend_store<D>(o, l, g + off, go + off, true);
}

// ---------------------------------------------------------------------------
// Triangle multiplicative update in fp32 (TriangleMultiplicationFull.forward,
// src/bioemu2/biomoa/ops/triangle_multiplication.py:89-99, which upcasts the
// projections before its einsum; TriangleMultiplicationCueq's default
// matmul_precision "ieee", :117).  The same wave tiling as gemm_f32_kernel:
// a wave owns a 32 x 32 block, weight rows in perm32 order as the A operand,
// so lane (n, h) ends with 16 consecutive output columns 16 h + u of row n.
// ---------------------------------------------------------------------------
// acc (+ acc2 with a second weight matrix) over K (a multiple of 8); arow and
// wrow / w2row already point at this lane's row and its k offset 4 h.
template <bool kTwo>
__device__ __forceinline__ void f32_block(const float* arow, const float* wrow, const float* w2row, int K, f32x16& acc,
                                          f32x16& acc2) {
  for (int k0 = 0; k0 < K; k0 += 8) {
    const f32x4 a4 = *reinterpret_cast<const f32x4*>(arow + k0);
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(wrow + k0);
    f32x4 v4;
    if (kTwo) v4 = *reinterpret_cast<const f32x4*>(w2row + k0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = mfma_f32(w4[e], a4[e], acc);
      if (kTwo) acc2 = mfma_f32(v4[e], a4[e], acc2);
    }
  }
}

// Gated, masked input projection p = (xn Wp^T) * sigmoid(xn Wg^T) * mask of
// the pair rows m = (b, r1, r2), written channel-major into the contraction's
// planes [b * 2D + c][i][k] (Np x Np each): (i, k) = (r1, r2) outgoing,
// (r2, r1) incoming, so both directions contract planes as C = A B^T.
__global__ __launch_bounds__(256) void trimul_proj_f32_kernel(const float* __restrict__ xn,
                                                              const float* __restrict__ wp,
                                                              const float* __restrict__ wg,
                                                              const uint8_t* __restrict__ mask,
                                                              float* __restrict__ planes, int N, int Np, int D,
                                                              long long M, int outgoing) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int nbc = 2 * D / 32;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  if (blk >= (M + 31) / 32 * nbc) return;   // no barriers in this kernel
  const long long m = blk / nbc * 32 + n;
  const int cb = (int)(blk % nbc);
  const bool mvalid = m < M;
  const size_t wr = (size_t)(cb * 32 + perm32(n)) * D + 4 * h;
  f32x16 acc = zero16(), acc2 = zero16();
  f32_block<true>(xn + (size_t)(mvalid ? m : 0) * D + 4 * h, wp + wr, wg + wr, D, acc, acc2);
  if (!mvalid) return;
  const float keep = mask[m] ? 1.f : 0.f;
  const long long b = m / ((long long)N * N), rr = m % ((long long)N * N);
  const int r1 = (int)(rr / N), r2 = (int)(rr % N);
  const int i = outgoing ? r1 : r2, k = outgoing ? r2 : r1;
  const size_t pl = (size_t)Np * Np;
  float* dst = planes + ((size_t)b * 2 * D + cb * 32 + 16 * h) * pl + (size_t)i * Np + k;
#pragma unroll
  for (int u = 0; u < 16; ++u) dst[(size_t)u * pl] = acc[u] / (1.0f + expf(-acc2[u])) * keep;
}

// o[b, i, j, d] = sum_k A[z][i][k] B[z][j][k], z = b * D + d (planes Np x Np,
// zero past N in k): a wave per 32 x 32 block of a plane; written pair-major.
__global__ __launch_bounds__(256) void trimul_contract_f32_kernel(const float* __restrict__ planes,
                                                                  float* __restrict__ o, int N, int Np, int Kp, int D) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int nb = Np / 32;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  if (blk >= (long long)nb * nb) return;   // no barriers in this kernel
  const int ib = (int)(blk / nb), jb = (int)(blk % nb);
  const int z = blockIdx.y, b = z / D, d = z % D;
  const size_t pl = (size_t)Np * Np;
  const float* A = planes + ((size_t)b * 2 * D + d) * pl;
  const float* Bm = A + (size_t)D * pl;
  f32x16 acc = zero16(), unused = zero16();
  const int i = ib * 32 + n;
  f32_block<false>(A + (size_t)i * Np + 4 * h, Bm + (size_t)(jb * 32 + perm32(n)) * Np + 4 * h, nullptr, Kp, acc,
                   unused);
  if (i >= N) return;
  float* dst = o + (((size_t)b * N + i) * N) * D + d;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int j = jb * 32 + 16 * h + u;
    if (j < N) dst[(size_t)j * D] = acc[u];
  }
}

// out = (on Wp_out^T) * gate (+ x): pair rows, D channels.
__global__ __launch_bounds__(256) void trimul_out_f32_kernel(const float* __restrict__ on,
                                                             const float* __restrict__ wo,
                                                             const float* __restrict__ gate, const float* x,
                                                             float* out, long long M, int D, int residual) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int nbc = D / 32;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  if (blk >= (M + 31) / 32 * nbc) return;   // no barriers in this kernel
  const long long m = blk / nbc * 32 + n;
  const int cb = (int)(blk % nbc);
  const bool mvalid = m < M;
  f32x16 acc = zero16(), unused = zero16();
  f32_block<false>(on + (size_t)(mvalid ? m : 0) * D + 4 * h, wo + (size_t)(cb * 32 + perm32(n)) * D + 4 * h, nullptr,
                   D, acc, unused);
  if (!mvalid) return;
  const size_t off = (size_t)m * D + cb * 32 + 16 * h;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    float v = acc[u] * gate[off + u];
    if (residual) v += x[off + u];
    out[off + u] = v;
  }
}

__global__ __launch_bounds__(256) void fill_zero_f32_kernel(float* __restrict__ p, long long count) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = 0.f;
}

int gemm_f32(int epi, const float* A, const float* W, const float* W2, const float* bias, const float* res, float* out,
             long long M, int K, int N, hipStream_t stream, const char* name, int T = 1, int ldT = 1) {
  if (K % 8 || N % 32 || M <= 0)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "%s: fp32 GEMM needs K %% 8 == 0 and N %% 32 == 0 (K=%d N=%d)", name, K,
                     N);
  const long long blocks = (M + 31) / 32 * (N / 32);
  const unsigned grid = (unsigned)((blocks + 3) / 4);
  KernelTimerScope timed(name, stream);
#define BIOEMU_GEMM_F32(E)                                                                                      \
  hipLaunchKernelGGL(gemm_f32_kernel<E>, dim3(grid), dim3(256), 0, stream, A, W, W2, bias, res, out, M, K, N, T, \
                     ldT)
  switch (epi) {
    case kGemmEpiStore: BIOEMU_GEMM_F32(kGemmEpiStore); break;
    case kGemmEpiSigmoid: BIOEMU_GEMM_F32(kGemmEpiSigmoid); break;
    case kGemmEpiSwiGLU: BIOEMU_GEMM_F32(kGemmEpiSwiGLU); break;
    case kGemmEpiStoreT: BIOEMU_GEMM_F32(kGemmEpiStoreT); break;
    default: BIOEMU_GEMM_F32(kGemmEpiResidual); break;
  }
#undef BIOEMU_GEMM_F32
  return check_launch(name);
}

int rows_ln_f32(const float* x, const float* g, const float* b, float* y, long long rows, int K, hipStream_t stream,
                const char* name, const float* x2 = nullptr, int K2 = 0) {
  KernelTimerScope timed(name, stream);
  hipLaunchKernelGGL(rows_ln_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, K, x2, K2, g, b,
                     y, rows);
  return check_launch(name);
}

// Bias rows: P pair rows = outer x nrows x ncols -> out[outer][head][row][col] with row stride ld.
int pair_proj_f32(const float* z, const float* g, const float* b, const float* w, float* out, long long P,
                  int nrows, int ncols, int ld, int H, int c_z, hipStream_t stream, const char* name) {
  const unsigned grid = (unsigned)((P + 255) / 256);
  KernelTimerScope timed(name, stream);
  if (c_z == 128)
    hipLaunchKernelGGL(pair_proj_f32_kernel<128>, dim3(grid), dim3(256), 0, stream, z, g, b, w, out, P, nrows, ncols,
                       ld, H);
  else if (c_z == 32)
    hipLaunchKernelGGL(pair_proj_f32_kernel<32>, dim3(grid), dim3(256), 0, stream, z, g, b, w, out, P, nrows, ncols,
                       ld, H);
  else if (c_z == 16)
    hipLaunchKernelGGL(pair_proj_f32_kernel<16>, dim3(grid), dim3(256), 0, stream, z, g, b, w, out, P, nrows, ncols,
                       ld, H);
  else
    return set_error(BIOEMU_ERR_UNSUPPORTED, "%s: c_z %d unsupported (16, 32 or 128)", name, c_z);
  return check_launch(name);
}

// Token-side projections shared by both attentions: optional LN, then q (+ q bias), k, v, sigmoid(g).
struct AttnF32Buffers {
  float *sn, *q, *k, *v, *g, *go, *bias;
};

// v is stored transposed per sequence ([sequence][c_s][ldv], keys contiguous): v_elems = sequences * c_s * ldv.
size_t attn_f32_layout(long long rows, int c_s, long long v_elems, long long bias_elems, bool norm,
                       AttnF32Buffers* buf, char* base) {
  size_t off = 0;
  auto take = [&](float** p, size_t elems) {
    if (buf) *p = reinterpret_cast<float*>(base + off);
    off += (size_t)round_up((int64_t)(elems * 4), 256);
  };
  AttnF32Buffers dummy;
  AttnF32Buffers* b = buf ? buf : &dummy;
  take(&b->sn, norm ? (size_t)rows * c_s : 0);
  take(&b->q, (size_t)rows * c_s);
  take(&b->k, (size_t)rows * c_s);
  take(&b->v, (size_t)v_elems);
  take(&b->g, (size_t)rows * c_s);
  take(&b->go, (size_t)rows * c_s);
  take(&b->bias, (size_t)bias_elems);
  return off;
}

int attn_f32_projections(const float* s, const float* norm_s_w, const float* norm_s_b, const float* w_qkv,
                         const float* q_bias, const float* w_g, AttnF32Buffers& buf, long long rows, int c_s,
                         int seq_len, int ldv, hipStream_t stream) {
  const float* src = s;
  int rc = 0;
  if (norm_s_w) {
    rc = rows_ln_f32(s, norm_s_w, norm_s_b, buf.sn, rows, c_s, stream, "f32_layernorm");
    src = buf.sn;
  }
  if (rc) return rc;
  if (c_s % 32) return set_error(BIOEMU_ERR_UNSUPPORTED, "f32 attention: c_s %d is not a multiple of 32", c_s);
  const long long blocks = (rows + 31) / 32 * (4 * (c_s / 32));
  KernelTimerScope timed("f32_proj_qkvg", stream);
  hipLaunchKernelGGL(qkvg_f32_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, stream, src, w_qkv, w_g, q_bias,
                     buf.q, buf.k, buf.v, buf.g, rows, c_s, seq_len, ldv);
  return check_launch("f32_proj_qkvg");
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_apb_f32_workspace_bytes(int64_t B, int64_t mult, int64_t N, int64_t c_s, int64_t H) {
  if (B <= 0 || mult <= 0 || N <= 0 || c_s <= 0 || H <= 0) return 0;
  const int64_t ld = round_up(N, 32);
  return attn_f32_layout(B * mult * N, (int)c_s, B * mult * c_s * ld, B * H * N * ld, true, nullptr, nullptr);
}

extern "C" int bioemu_apb_fwd_f32(const float* s, const float* z, const uint8_t* mask, const float* norm_s_w,
                                  const float* norm_s_b, const float* w_qkv, const float* q_bias, const float* w_g,
                                  const float* norm_z_w, const float* norm_z_b, const float* w_z, const float* w_o,
                                  float* out, void* workspace, size_t workspace_bytes, int64_t B, int64_t mult,
                                  int64_t N, int64_t c_s, int64_t c_z, int64_t H, int residual, hipStream_t stream) {
  if (H <= 0 || c_s % H || (c_s / H != 24 && c_s / H != 32) || c_s % 32 || (c_z != 128 && c_z != 32 && c_z != 16))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "apb_f32: supported are head dim 24 or 32 with c_s a multiple of 32, c_z in {16, 32, 128} "
                     "(got c_s=%lld H=%lld c_z=%lld)", (long long)c_s, (long long)H, (long long)c_z);
  if (B <= 0 || mult <= 0 || N <= 0 || B * mult > 65535 || H > 65535)
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb_f32: bad shape B=%lld M=%lld N=%lld", (long long)B,
                     (long long)mult, (long long)N);
  if (!s || !z || !mask || !w_qkv || !q_bias || !w_g || !norm_z_w || !w_z || !w_o || !out || !workspace ||
      (norm_s_w == nullptr) != (norm_s_b == nullptr))
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb_f32: null pointer argument");
  if (!aligned16(s) || !aligned16(z) || !aligned16(out) || !aligned16(w_qkv) || !aligned16(w_g) || !aligned16(w_o) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb_f32: tensors must be 16-byte aligned");
  if (out == s && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb_f32: out may alias s only with residual=1");
  if (workspace_bytes < bioemu_apb_f32_workspace_bytes(B, mult, N, c_s, H))
    return set_error(BIOEMU_ERR_WORKSPACE, "apb_f32: workspace too small");
  const long long rows = B * mult * N;
  AttnF32Buffers buf;
  const int ldb = (int)round_up(N, 32);
  attn_f32_layout(rows, (int)c_s, B * mult * c_s * ldb, B * H * N * ldb, true, &buf, static_cast<char*>(workspace));
  int rc = attn_f32_projections(s, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, buf, rows, (int)c_s, (int)N, ldb, stream);
  if (rc) return rc;
  rc = pair_proj_f32(z, norm_z_w, norm_z_b, w_z, buf.bias, B * N * N, (int)N, (int)N, ldb, (int)H, (int)c_z, stream,
                     "f32_pair_bias");
  if (rc) return rc;
  {
    KernelTimerScope timed("f32_attention", stream);
    const dim3 grid((unsigned)((N + 127) / 128), (unsigned)H, (unsigned)(B * mult));
    const int d = (int)(c_s / H);
    const float rsq = 1.0f / std::sqrt((float)d);
    if (d == 24)
      hipLaunchKernelGGL(attn_f32_kernel<24>, grid, dim3(256), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, mask,
                         buf.go, (int)N, ldb, (int)H, (int)c_s, (int)mult, rsq, 0);
    else
      hipLaunchKernelGGL(attn_f32_kernel<32>, grid, dim3(256), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, mask,
                         buf.go, (int)N, ldb, (int)H, (int)c_s, (int)mult, rsq, 0);
  }
  rc = check_launch("f32_attention");
  if (rc) return rc;
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, buf.go, w_o, nullptr, nullptr, s, out, rows, (int)c_s,
                  (int)c_s, stream, "f32_proj_o");
}

extern "C" size_t bioemu_swa_f32_workspace_bytes(int64_t B, int64_t mult, int64_t NW, int64_t W, int64_t H,
                                                 int64_t c_s, int64_t heads) {
  if (B <= 0 || mult <= 0 || NW <= 0 || W != 32 || H <= 0 || c_s <= 0 || heads <= 0) return 0;
  return attn_f32_layout(B * mult * NW * W, (int)c_s, B * mult * NW * W * c_s, B * NW * heads * W * H, true, nullptr,
                         nullptr);
}

extern "C" int bioemu_swa_fwd_f32(const float* s, const float* z, const uint8_t* mask, const float* norm_s_w,
                                  const float* norm_s_b, const float* w_qkv, const float* q_bias, const float* w_g,
                                  const float* norm_z_w, const float* norm_z_b, const float* w_z, const float* w_o,
                                  float* out, void* workspace, size_t workspace_bytes, int64_t B, int64_t mult,
                                  int64_t NW, int64_t W, int64_t H, int64_t c_s, int64_t c_z, int64_t heads,
                                  int residual, hipStream_t stream) {
  if (W != 32 || H < W || (H - W) % 2 || H % 32 || heads <= 0 || c_s % heads || c_s / heads != 32 || c_s % 32 ||
      (c_z != 16 && c_z != 32 && c_z != 128))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "swa_f32: supported are W=32, H a multiple of 32 (H >= W), head dim 32, c_z in {16, 32, 128} "
                     "(got W=%lld H=%lld c_s=%lld heads=%lld c_z=%lld)", (long long)W, (long long)H, (long long)c_s,
                     (long long)heads, (long long)c_z);
  if (B <= 0 || mult <= 0 || NW <= 0 || B * mult > 65535 || NW > 65535)
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa_f32: bad shape B=%lld M=%lld NW=%lld", (long long)B,
                     (long long)mult, (long long)NW);
  if (!s || !z || !mask || !w_qkv || !q_bias || !w_g || !norm_z_w || !w_z || !w_o || !out || !workspace ||
      (norm_s_w == nullptr) != (norm_s_b == nullptr))
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa_f32: null pointer argument");
  if (!aligned16(s) || !aligned16(z) || !aligned16(out) || !aligned16(w_qkv) || !aligned16(w_g) || !aligned16(w_o) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa_f32: tensors must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(mask) & 3)
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa_f32: mask must be 4-byte aligned (it is read 4 keys at a time)");
  if (out == s && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa_f32: out may alias s only with residual=1");
  if (workspace_bytes < bioemu_swa_f32_workspace_bytes(B, mult, NW, W, H, c_s, heads))
    return set_error(BIOEMU_ERR_WORKSPACE, "swa_f32: workspace too small");
  const long long rows = B * mult * NW * W;
  AttnF32Buffers buf;
  attn_f32_layout(rows, (int)c_s, rows * c_s, B * NW * heads * W * H, true, &buf, static_cast<char*>(workspace));
  int rc = attn_f32_projections(s, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, buf, rows, (int)c_s, (int)(NW * W),
                                (int)(NW * W), stream);
  if (rc) return rc;
  rc = pair_proj_f32(z, norm_z_w, norm_z_b, w_z, buf.bias, B * NW * W * H, (int)W, (int)H, (int)H, (int)heads,
                     (int)c_z, stream, "f32_swa_pair_bias");
  if (rc) return rc;
  {
    KernelTimerScope timed("f32_swa_attention", stream);
    hipLaunchKernelGGL(swa_attn_f32_kernel, dim3((unsigned)NW, (unsigned)((heads + 3) / 4), (unsigned)(B * mult)),
                       dim3(256), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, mask, buf.go, (int)NW, (int)H,
                       (int)heads, (int)c_s, (int)mult, 1.0f / std::sqrt(32.0f));
  }
  rc = check_launch("f32_swa_attention");
  if (rc) return rc;
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, buf.go, w_o, nullptr, nullptr, s, out, rows, (int)c_s,
                  (int)c_s, stream, "f32_proj_o");
}

// out = (res +) Transition(x) over M rows; res may differ from x (the trunk's unconditional branch adds the
// transition of LN(z_init) to z_init).  workspace: the LN rows [M][Dc], then the hidden rows [M][hidden].
static int transition_f32_res(const float* x, const float* res, const float* norm_w, const float* norm_b,
                              const float* fc1_w, const float* fc2_w, const float* fc3_w, float* out, void* workspace,
                              int64_t M, int64_t Dc, int64_t hidden, int64_t out_dim, int use_norm, int residual,
                              hipStream_t stream) {
  float* xn = static_cast<float*>(workspace);
  float* hbuf = reinterpret_cast<float*>(static_cast<char*>(workspace) + round_up(M * Dc * 4, 256));
  const float* src = x;
  int rc = 0;
  if (use_norm) {
    rc = rows_ln_f32(x, norm_w, norm_b, xn, M, (int)Dc, stream, "f32_layernorm");
    src = xn;
  }
  if (!rc)
    rc = gemm_f32(kGemmEpiSwiGLU, src, fc1_w, fc2_w, nullptr, nullptr, hbuf, M, (int)Dc, (int)hidden, stream,
                  "f32_transition_swiglu");
  if (rc) return rc;
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, hbuf, fc3_w, nullptr, nullptr, res, out, M,
                  (int)hidden, (int)out_dim, stream, "f32_transition_out");
}

extern "C" size_t bioemu_transition_f32_workspace_bytes(int64_t M, int64_t Dc, int64_t hidden) {
  if (M <= 0 || Dc <= 0 || hidden <= 0) return 0;
  return (size_t)round_up(M * Dc * 4, 256) + (size_t)round_up(M * hidden * 4, 256);
}

extern "C" int bioemu_transition_fwd_f32(const float* x, const float* norm_w, const float* norm_b, const float* fc1_w,
                                         const float* fc2_w, const float* fc3_w, float* out, void* workspace,
                                         size_t workspace_bytes, int64_t M, int64_t Dc, int64_t hidden,
                                         int64_t out_dim, int use_norm, int residual, hipStream_t stream) {
  if (M <= 0 || Dc <= 0 || Dc % 8 || hidden <= 0 || hidden % 32 || out_dim <= 0 || out_dim % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "transition_f32: dim %lld / hidden %lld / out_dim %lld unsupported (dim a multiple of 8, hidden "
                     "and out_dim multiples of 32)", (long long)Dc, (long long)hidden, (long long)out_dim);
  if (residual && out_dim != Dc)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_f32: residual=1 needs out_dim == dim");
  if (!x || !fc1_w || !fc2_w || !fc3_w || !out || !workspace || (use_norm && !norm_w))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_f32: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(fc1_w) || !aligned16(fc2_w) || !aligned16(fc3_w) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_f32: tensors must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_f32: out may alias x only with residual=1");
  if (workspace_bytes < bioemu_transition_f32_workspace_bytes(M, Dc, hidden))
    return set_error(BIOEMU_ERR_WORKSPACE, "transition_f32: workspace too small");
  return transition_f32_res(x, x, norm_w, norm_b, fc1_w, fc2_w, fc3_w, out, workspace, M, Dc, hidden, out_dim,
                            use_norm, residual, stream);
}

extern "C" size_t bioemu_pair_cond_f32_workspace_bytes(int64_t P, int64_t token_z, int64_t c_rel) {
  if (P <= 0 || token_z <= 0 || c_rel < 0) return 0;
  return (size_t)round_up(P * (token_z + c_rel) * 4, 256);
}

extern "C" int bioemu_pair_cond_proj_fwd_f32(const float* z_trunk, const float* rel, const float* ln_w,
                                             const float* ln_b, const float* w, float* out, void* workspace,
                                             size_t workspace_bytes, int64_t P, int64_t token_z, int64_t c_rel,
                                             int64_t a_z, hipStream_t stream) {
  if (token_z <= 0 || c_rel < 0 || (token_z + c_rel) % 8 || a_z <= 0 || a_z % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "pair_cond_f32: token_z + c_rel must be a multiple of 8 and a_z of 32 (got %lld + %lld, %lld)",
                     (long long)token_z, (long long)c_rel, (long long)a_z);
  if (P <= 0) return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond_f32: bad row count %lld", (long long)P);
  if (!z_trunk || (c_rel && !rel) || !ln_w || !ln_b || !w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond_f32: null pointer argument");
  if (!aligned16(w) || !aligned16(out) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond_f32: tensors must be 16-byte aligned");
  if (workspace_bytes < bioemu_pair_cond_f32_workspace_bytes(P, token_z, c_rel))
    return set_error(BIOEMU_ERR_WORKSPACE, "pair_cond_f32: workspace too small");
  float* xn = static_cast<float*>(workspace);
  int rc = rows_ln_f32(z_trunk, ln_w, ln_b, xn, P, (int)token_z, stream, "f32_pair_cond_layernorm", rel, (int)c_rel);
  if (rc) return rc;
  return gemm_f32(kGemmEpiStore, xn, w, nullptr, nullptr, nullptr, out, P, (int)(token_z + c_rel), (int)a_z, stream,
                  "f32_pair_cond_proj");
}

// ---------------------------------------------------------------------------
// Triangle multiplicative update, fp32 arithmetic.
// ---------------------------------------------------------------------------
static int64_t trimul_f32_np(int64_t N) { return round_up(N, 32); }

extern "C" size_t bioemu_trimul_f32_workspace_bytes(int64_t B, int64_t N, int64_t Dc) {
  if (B <= 0 || N <= 0 || Dc <= 0 || Dc % 32) return 0;
  const size_t P = (size_t)B * N * N, Np = (size_t)trimul_f32_np(N);
  // xn (then LN_out(o)), the output gate, o: [P][D] each; the planes [B][2D][Np][Np]
  return (size_t)round_up(P * Dc * 4, 256) * 3 + (size_t)round_up(B * 2 * Dc * Np * Np * 4, 256);
}

extern "C" int bioemu_trimul_fwd_f32(const float* x, const uint8_t* mask, const float* norm_in_w,
                                     const float* norm_in_b, const float* p_in_w, const float* g_in_w,
                                     const float* norm_out_w, const float* norm_out_b, const float* p_out_w,
                                     const float* g_out_w, float* out, void* workspace, size_t workspace_bytes,
                                     int64_t B, int64_t N, int64_t Dc, int outgoing, int residual,
                                     hipStream_t stream) {
  if (Dc <= 0 || Dc % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "trimul_f32: dim must be a multiple of 32 (got %lld)", (long long)Dc);
  if (B <= 0 || N <= 0 || B * Dc > 65535 || N > 16384)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul_f32: bad shape B=%lld N=%lld (B * dim <= 65535)", (long long)B,
                     (long long)N);
  if (!x || !mask || !norm_in_w || !norm_in_b || !p_in_w || !g_in_w || !norm_out_w || !norm_out_b || !p_out_w ||
      !g_out_w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul_f32: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(p_in_w) || !aligned16(g_in_w) || !aligned16(p_out_w) ||
      !aligned16(g_out_w) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul_f32: tensors must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul_f32: out may alias x only with residual=1");
  if (workspace_bytes < bioemu_trimul_f32_workspace_bytes(B, N, Dc))
    return set_error(BIOEMU_ERR_WORKSPACE, "trimul_f32: workspace too small");
  const long long P = B * N * N;
  const int64_t Np = trimul_f32_np(N);
  const int D = (int)Dc;
  char* p = static_cast<char*>(workspace);
  float* xn = reinterpret_cast<float*>(p);
  p += round_up(P * Dc * 4, 256);
  float* gate = reinterpret_cast<float*>(p);
  p += round_up(P * Dc * 4, 256);
  float* o = reinterpret_cast<float*>(p);
  p += round_up(P * Dc * 4, 256);
  float* planes = reinterpret_cast<float*>(p);
  const long long plane_count = B * 2 * Dc * Np * Np;

  int rc = rows_ln_f32(x, norm_in_w, norm_in_b, xn, P, D, stream, "f32_trimul_ln_in");
  if (rc) return rc;
  {
    KernelTimerScope timed("f32_fill", stream);
    hipLaunchKernelGGL(fill_zero_f32_kernel, dim3((unsigned)((plane_count + 255) / 256)), dim3(256), 0, stream,
                       planes, plane_count);
  }
  if ((rc = check_launch("f32_fill"))) return rc;
  {
    const long long blocks = (P + 31) / 32 * (2 * D / 32);
    KernelTimerScope timed("f32_trimul_proj", stream);
    hipLaunchKernelGGL(trimul_proj_f32_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, stream, xn, p_in_w,
                       g_in_w, mask, planes, (int)N, (int)Np, D, P, outgoing);
  }
  if ((rc = check_launch("f32_trimul_proj"))) return rc;
  rc = gemm_f32(kGemmEpiSigmoid, xn, g_out_w, nullptr, nullptr, nullptr, gate, P, D, D, stream, "f32_trimul_gate");
  if (rc) return rc;
  {
    const long long nb = Np / 32;
    KernelTimerScope timed("f32_trimul_contract", stream);
    hipLaunchKernelGGL(trimul_contract_f32_kernel, dim3((unsigned)((nb * nb + 3) / 4), (unsigned)(B * Dc)), dim3(256), 0,
                       stream, planes, o, (int)N, (int)Np, (int)round_up(N, 8), D);
  }
  if ((rc = check_launch("f32_trimul_contract"))) return rc;
  rc = rows_ln_f32(o, norm_out_w, norm_out_b, xn, P, D, stream, "f32_trimul_ln_out");
  if (rc) return rc;
  {
    const long long blocks = (P + 31) / 32 * (D / 32);
    KernelTimerScope timed("f32_trimul_out", stream);
    hipLaunchKernelGGL(trimul_out_f32_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, stream, xn, p_out_w,
                       gate, x, out, P, D, residual);
  }
  return check_launch("f32_trimul_out");
}

// ---------------------------------------------------------------------------
// OuterProductMean, fp32 arithmetic (outer_product_mean.py:45-75 with autocast
// off: LayerNorm, proj_ab, the masked contraction over the MSA rows, the mean
// and proj_o all in fp32).
//   mn = LN(m);  [a | b] = mn W_ab^T, zeroed where mask[b,s,n] == 0
//   aT[b][(n, c)][s], bT[b][(n, d)][s]   (s contiguous, zero for s >= S)
//   Y[(b, i, j)][c * C_H + d] = sum_s aT[b][(i, c)][s] bT[b][(j, d)][s] * inv[b]
//   out = Y W_o^T + b_o (+ z)
// A 32 x 32 block of the contraction (rows (i, c), columns (j, d)) is exactly
// one pair's C_H x C_H outer-product matrix (C_H = 32), which the epilogue
// stores as that pair's row of Y.  inv[b] = 1 / max(valid rows, 1) with a
// [B,S,N] mask, 1 for the broadcast [B,N] one (mean_rows = 0).
// ---------------------------------------------------------------------------
namespace bioemu {
namespace {

constexpr int kOpmCH = 32;

// The proj_ab block of 32 rows m = (b, s, n) x 32 output channels (cb = 0: a, 1: b),
// masked and stored transposed into aT / bT.
__global__ __launch_bounds__(256) void opm_proj_f32_kernel(const float* __restrict__ mn, const float* __restrict__ wab,
                                                           const uint8_t* __restrict__ mask, float* __restrict__ aT,
                                                           float* __restrict__ bT, int S, int N, int Sp, int cin,
                                                           long long M) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  if (blk >= (M + 31) / 32 * 2) return;   // no barriers in this kernel
  const long long m = blk / 2 * 32 + n;
  const int cb = (int)(blk % 2);
  const bool mvalid = m < M;
  f32x16 acc = zero16(), unused = zero16();
  f32_block<false>(mn + (size_t)(mvalid ? m : 0) * cin + 4 * h, wab + (size_t)(cb * 32 + perm32(n)) * cin + 4 * h,
                   nullptr, cin, acc, unused);
  if (!mvalid) return;
  const float keep = mask[m] ? 1.f : 0.f;
  const long long b = m / ((long long)S * N), r = m % ((long long)S * N);
  const int s = (int)(r / N), tok = (int)(r % N);
  float* dst = (cb ? bT : aT) + (((size_t)b * N + tok) * kOpmCH + 16 * h) * Sp + s;
#pragma unroll
  for (int u = 0; u < 16; ++u) dst[(size_t)u * Sp] = acc[u] * keep;
}

// inv[b] = 1 / max(#rows s with any mask[b, s, :], 1), or 1 when !mean_rows.  One workgroup per batch.
__global__ __launch_bounds__(256) void opm_inv_f32_kernel(const uint8_t* __restrict__ mask, float* __restrict__ inv,
                                                          int S, int N, int mean_rows) {
  __shared__ int cnt;
  if (threadIdx.x == 0) cnt = 0;
  __syncthreads();
  const uint8_t* mb = mask + (size_t)blockIdx.x * S * N;
  int local = 0;
  for (int s = threadIdx.x; s < S; s += blockDim.x) {
    bool any = false;
    for (int t = 0; t < N && !any; ++t) any = mb[(size_t)s * N + t] != 0;
    local += any;
  }
  atomicAdd(&cnt, local);
  __syncthreads();
  if (threadIdx.x == 0) inv[blockIdx.x] = mean_rows ? 1.0f / (float)max(cnt, 1) : 1.0f;
}

// One wave per pair (i, j) of batch blockIdx.y: Y row = the 32 x 32 block (i, j) of aT bT^T, times inv[b].
__global__ __launch_bounds__(256) void opm_contract_f32_kernel(const float* __restrict__ aT, const float* __restrict__ bT,
                                                               const float* __restrict__ inv, float* __restrict__ Y,
                                                               int N, int Sp) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const long long pair = (long long)blockIdx.x * 4 + wave;
  if (pair >= (long long)N * N) return;   // no barriers in this kernel
  const int i = (int)(pair / N), j = (int)(pair % N), b = blockIdx.y;
  const float* A = aT + (((size_t)b * N + i) * kOpmCH + n) * Sp + 4 * h;
  const float* Bm = bT + (((size_t)b * N + j) * kOpmCH + perm32(n)) * Sp + 4 * h;
  f32x16 acc = zero16(), unused = zero16();
  f32_block<false>(A, Bm, nullptr, Sp, acc, unused);
  // lane (n, h): row c = n, register u <-> column d = 16 h + u
  const float scale = inv[b];
  float* dst = Y + (((size_t)b * N + i) * N + j) * (kOpmCH * kOpmCH) + n * kOpmCH + 16 * h;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 o4;
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = acc[4 * q + e] * scale;
    *reinterpret_cast<f32x4*>(dst + 4 * q) = o4;
  }
}

struct OpmF32Layout {
  size_t mn, aT, bT, inv, Y, total;
};

OpmF32Layout opm_f32_layout(int64_t B, int64_t S, int64_t N, int64_t c_in) {
  OpmF32Layout L;
  const size_t Sp = (size_t)round_up(S, 8);
  size_t off = 0;
  L.mn = off;
  off += round_up((size_t)B * S * N * c_in * 4, 256);
  L.aT = off;
  off += round_up((size_t)B * N * kOpmCH * Sp * 4, 256);
  L.bT = off;
  off += round_up((size_t)B * N * kOpmCH * Sp * 4, 256);
  L.inv = off;
  off += round_up((size_t)B * 4, 256);
  L.Y = off;
  off += round_up((size_t)B * N * N * kOpmCH * kOpmCH * 4, 256);
  L.total = off;
  return L;
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_opm_f32_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_in, int64_t c_hidden) {
  if (B <= 0 || S <= 0 || N <= 0 || c_in <= 0 || c_hidden != kOpmCH) return 0;
  return opm_f32_layout(B, S, N, c_in).total;
}

extern "C" int bioemu_opm_fwd_f32(const float* m, const uint8_t* mask, int mean_rows, const float* norm_w,
                                  const float* norm_b, const float* w_ab, const float* w_o, const float* b_o,
                                  const float* z_res, float* out, void* workspace, size_t workspace_bytes, int64_t B,
                                  int64_t S, int64_t N, int64_t c_in, int64_t c_hidden, int64_t c_out,
                                  hipStream_t stream) {
  if (c_hidden != kOpmCH || c_in <= 0 || c_in % 8 || c_out <= 0 || c_out % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "opm_f32: c_hidden must be 32, c_in a multiple of 8 and c_out of 32 (got %lld/%lld/%lld)",
                     (long long)c_in, (long long)c_hidden, (long long)c_out);
  if (B <= 0 || S <= 0 || N <= 0 || B > 65535 || N > 16384 || S > (1 << 24))
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm_f32: bad shape B=%lld S=%lld N=%lld", (long long)B, (long long)S,
                     (long long)N);
  if (!m || !mask || !norm_w || !norm_b || !w_ab || !w_o || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm_f32: null pointer argument");
  if (!aligned16(m) || !aligned16(w_ab) || !aligned16(w_o) || !aligned16(out) || !aligned16(workspace) ||
      (z_res && !aligned16(z_res)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm_f32: tensors must be 16-byte aligned");
  const OpmF32Layout L = opm_f32_layout(B, S, N, c_in);
  if (workspace_bytes < L.total) return set_error(BIOEMU_ERR_WORKSPACE, "opm_f32: workspace too small");
  char* p = static_cast<char*>(workspace);
  float* mn = reinterpret_cast<float*>(p + L.mn);
  float* aT = reinterpret_cast<float*>(p + L.aT);
  float* bT = reinterpret_cast<float*>(p + L.bT);
  float* inv = reinterpret_cast<float*>(p + L.inv);
  float* Y = reinterpret_cast<float*>(p + L.Y);
  const long long M = B * S * N;
  const int Sp = (int)round_up(S, 8);

  int rc = rows_ln_f32(m, norm_w, norm_b, mn, M, (int)c_in, stream, "f32_opm_layernorm");
  if (rc) return rc;
  {
    // aT and bT are adjacent: one fill zeroes both (the rows s in [S, Sp) stay zero)
    const long long count = (long long)((L.bT - L.aT) / 4) * 2;
    KernelTimerScope timed("f32_fill", stream);
    hipLaunchKernelGGL(fill_zero_f32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream, aT, count);
  }
  if ((rc = check_launch("f32_fill"))) return rc;
  {
    const long long blocks = (M + 31) / 32 * 2;
    KernelTimerScope timed("f32_opm_proj", stream);
    hipLaunchKernelGGL(opm_proj_f32_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, stream, mn, w_ab, mask,
                       aT, bT, (int)S, (int)N, Sp, (int)c_in, M);
  }
  if ((rc = check_launch("f32_opm_proj"))) return rc;
  {
    KernelTimerScope timed("f32_opm_count", stream);
    hipLaunchKernelGGL(opm_inv_f32_kernel, dim3((unsigned)B), dim3(256), 0, stream, mask, inv, (int)S, (int)N,
                       mean_rows);
  }
  if ((rc = check_launch("f32_opm_count"))) return rc;
  {
    const long long pairs = N * N;
    KernelTimerScope timed("f32_opm_contract", stream);
    hipLaunchKernelGGL(opm_contract_f32_kernel, dim3((unsigned)((pairs + 3) / 4), (unsigned)B), dim3(256), 0, stream,
                       aT, bT, inv, Y, (int)N, Sp);
  }
  if ((rc = check_launch("f32_opm_contract"))) return rc;
  return gemm_f32(z_res ? kGemmEpiResidual : kGemmEpiStore, Y, w_o, nullptr, b_o, z_res, out, B * N * N,
                  kOpmCH * kOpmCH, (int)c_out, stream, "f32_opm_out");
}

// ---------------------------------------------------------------------------
// Pair-weighted averaging, fp32 arithmetic (pair_weighted_averaging.py:125-154
// with autocast off).
//   mn = LN_m(m);  vT[b][h][(s, d)][j] = (mn W_m^T)[b, s, j, h*32 + d]   (j contiguous)
//   g = sigmoid(mn W_g^T);  logits[b][h][i][j] = LN_z(z[b, i, j]) W_z^T [h]
//   w = softmax_j(logits, masked keys -> -1e6)
//   go[b, s, i, h*32 + d] = g * sum_j w[b][h][i][j] vT[b][h][(s, d)][j]
//   out = go W_o^T (+ m)
// Keys are padded to Np8 = N rounded up to 8 with zero weights and zero v.
// ---------------------------------------------------------------------------
namespace bioemu {
namespace {

constexpr int kPwaCH = 32;

// v block of 32 rows m = (b, s, j) x 32 channels (head hd = cb), stored transposed into vT.
__global__ __launch_bounds__(256) void pwa_v_f32_kernel(const float* __restrict__ mn, const float* __restrict__ wm,
                                                        float* __restrict__ vT, int S, int N, int Np8, int cm, int H,
                                                        long long M) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  if (blk >= (M + 31) / 32 * H) return;   // no barriers in this kernel
  const long long m = blk / H * 32 + n;
  const int hd = (int)(blk % H);
  const bool mvalid = m < M;
  f32x16 acc = zero16(), unused = zero16();
  f32_block<false>(mn + (size_t)(mvalid ? m : 0) * cm + 4 * h, wm + (size_t)(hd * 32 + perm32(n)) * cm + 4 * h,
                   nullptr, cm, acc, unused);
  if (!mvalid) return;
  const long long b = m / ((long long)S * N), r = m % ((long long)S * N);
  const int s = (int)(r / N), j = (int)(r % N);
  float* dst = vT + ((((size_t)b * H + hd) * S + s) * kPwaCH + 16 * h) * Np8 + j;
#pragma unroll
  for (int u = 0; u < 16; ++u) dst[(size_t)u * Np8] = acc[u];
}

// In place over logits rows [b][h][i][0, Np8): masked keys -> -inf_value, softmax over the N keys, 0 past N.
// One wave per row.
__global__ __launch_bounds__(256) void pwa_softmax_f32_kernel(float* __restrict__ lg, const uint8_t* __restrict__ mask,
                                                              int N, int Np8, int H, long long rows, float neg) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const long long bh = row / N;
  const int i = (int)(row % N);
  const long long b = bh / H;
  float* x = lg + (size_t)row * Np8;
  const uint8_t* mk = mask + ((size_t)b * N + i) * N;
  float mx = -INFINITY;
  for (int j = lane; j < N; j += 64) {
    const float v = mk[j] ? x[j] : neg;
    x[j] = v;
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float sum = 0.f;
  for (int j = lane; j < N; j += 64) {
    const float e = expf(x[j] - mx);
    x[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  const float r = 1.0f / sum;
  for (int j = lane; j < Np8; j += 64) x[j] = j < N ? x[j] * r : 0.f;
}

// One wave per 32 x 32 block (query rows i, columns (s, d) = one MSA row s) of head hd = blockIdx.y % H:
// go[b, s, i, hd*32 + d] = g[same] * sum_j w[b][hd][i][j] vT[b][hd][(s, d)][j].
__global__ __launch_bounds__(256) void pwa_avg_f32_kernel(const float* __restrict__ w, const float* __restrict__ vT,
                                                          const float* __restrict__ g, float* __restrict__ go, int S,
                                                          int N, int Np8, int H) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int nib = (N + 31) / 32;
  const long long blk = (long long)blockIdx.x * 4 + wave;
  if (blk >= (long long)nib * S) return;   // no barriers in this kernel
  const int ib = (int)(blk % nib), s = (int)(blk / nib);
  const int bh = blockIdx.y, b = bh / H, hd = bh % H;
  const int i = ib * 32 + n;
  const bool ivalid = i < N;
  const float* A = w + ((size_t)bh * N + (ivalid ? i : 0)) * Np8 + 4 * h;
  const float* Bm = vT + (((size_t)bh * S + s) * kPwaCH + perm32(n)) * Np8 + 4 * h;
  f32x16 acc = zero16(), unused = zero16();
  f32_block<false>(A, Bm, nullptr, Np8, acc, unused);
  if (!ivalid) return;
  // lane (n, h): query i, register u <-> d = 16 h + u
  const size_t off = (((size_t)b * S + s) * N + i) * (size_t)(H * kPwaCH) + hd * kPwaCH + 16 * h;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 g4 = *reinterpret_cast<const f32x4*>(g + off + 4 * q);
    f32x4 o4;
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = acc[4 * q + e] * g4[e];
    *reinterpret_cast<f32x4*>(go + off + 4 * q) = o4;
  }
}

struct PwaF32Layout {
  size_t mn, vT, g, go, lg, total;
};

PwaF32Layout pwa_f32_layout(int64_t B, int64_t S, int64_t N, int64_t c_m, int64_t H) {
  PwaF32Layout L;
  const size_t Np8 = (size_t)round_up(N, 8), rows = (size_t)B * S * N, hc = (size_t)H * kPwaCH;
  size_t off = 0;
  L.mn = off;
  off += round_up(rows * c_m * 4, 256);
  L.vT = off;
  off += round_up((size_t)B * H * S * kPwaCH * Np8 * 4, 256);
  L.g = off;
  off += round_up(rows * hc * 4, 256);
  L.go = off;
  off += round_up(rows * hc * 4, 256);
  L.lg = off;
  off += round_up((size_t)B * H * N * Np8 * 4, 256);
  L.total = off;
  return L;
}

}  // namespace
}  // namespace bioemu

extern "C" size_t bioemu_pwa_f32_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_m, int64_t c_h, int64_t H) {
  if (B <= 0 || S <= 0 || N <= 0 || c_m <= 0 || c_h != kPwaCH || H <= 0) return 0;
  return pwa_f32_layout(B, S, N, c_m, H).total;
}

extern "C" int bioemu_pwa_fwd_f32(const float* m, const float* z, const uint8_t* mask, const float* norm_m_w,
                                  const float* norm_m_b, const float* norm_z_w, const float* norm_z_b,
                                  const float* w_m, const float* w_g, const float* w_z, const float* w_o, float* out,
                                  void* workspace, size_t workspace_bytes, int64_t B, int64_t S, int64_t N,
                                  int64_t c_m, int64_t c_z, int64_t c_h, int64_t H, float inf, int residual,
                                  hipStream_t stream) {
  if (c_h != kPwaCH || c_m <= 0 || c_m % 32 || H <= 0 || H > 64 || (c_z != 128 && c_z != 32 && c_z != 16))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "pwa_f32: c_h must be 32, c_m a multiple of 32, c_z 16, 32 or 128 (got c_m=%lld c_z=%lld c_h=%lld "
                     "H=%lld)", (long long)c_m, (long long)c_z, (long long)c_h, (long long)H);
  if (B <= 0 || S <= 0 || N <= 0 || B * H > 65535 || N > 16384)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa_f32: bad shape B=%lld S=%lld N=%lld", (long long)B, (long long)S,
                     (long long)N);
  if (!m || !z || !mask || !norm_m_w || !norm_z_w || !w_m || !w_g || !w_z || !w_o || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa_f32: null pointer argument");
  if (!aligned16(m) || !aligned16(z) || !aligned16(w_m) || !aligned16(w_g) || !aligned16(w_o) || !aligned16(out) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa_f32: tensors must be 16-byte aligned");
  if (out == m && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa_f32: out may alias m only with residual=1");
  const PwaF32Layout L = pwa_f32_layout(B, S, N, c_m, H);
  if (workspace_bytes < L.total) return set_error(BIOEMU_ERR_WORKSPACE, "pwa_f32: workspace too small");
  char* p = static_cast<char*>(workspace);
  float* mn = reinterpret_cast<float*>(p + L.mn);
  float* vT = reinterpret_cast<float*>(p + L.vT);
  float* g = reinterpret_cast<float*>(p + L.g);
  float* go = reinterpret_cast<float*>(p + L.go);
  float* lg = reinterpret_cast<float*>(p + L.lg);
  const long long M = B * S * N;
  const int Np8 = (int)round_up(N, 8), hc = (int)(H * kPwaCH);

  int rc = rows_ln_f32(m, norm_m_w, norm_m_b, mn, M, (int)c_m, stream, "f32_pwa_layernorm");
  if (rc) return rc;
  {
    const long long count = (long long)((L.g - L.vT) / 4);   // vT, zero past N in j
    KernelTimerScope timed("f32_fill", stream);
    hipLaunchKernelGGL(fill_zero_f32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream, vT, count);
  }
  if ((rc = check_launch("f32_fill"))) return rc;
  {
    const long long blocks = (M + 31) / 32 * H;
    KernelTimerScope timed("f32_pwa_v", stream);
    hipLaunchKernelGGL(pwa_v_f32_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, stream, mn, w_m, vT,
                       (int)S, (int)N, Np8, (int)c_m, (int)H, M);
  }
  if ((rc = check_launch("f32_pwa_v"))) return rc;
  rc = gemm_f32(kGemmEpiSigmoid, mn, w_g, nullptr, nullptr, nullptr, g, M, (int)c_m, hc, stream, "f32_pwa_gate");
  if (rc) return rc;
  rc = pair_proj_f32(z, norm_z_w, norm_z_b, w_z, lg, B * N * N, (int)N, (int)N, Np8, (int)H, (int)c_z, stream,
                     "f32_pwa_logits");
  if (rc) return rc;
  {
    const long long rows = B * H * N;
    KernelTimerScope timed("f32_pwa_softmax", stream);
    hipLaunchKernelGGL(pwa_softmax_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, lg, mask,
                       (int)N, Np8, (int)H, rows, -inf);
  }
  if ((rc = check_launch("f32_pwa_softmax"))) return rc;
  {
    const long long blocks = (N + 31) / 32 * S;
    KernelTimerScope timed("f32_pwa_average", stream);
    hipLaunchKernelGGL(pwa_avg_f32_kernel, dim3((unsigned)((blocks + 3) / 4), (unsigned)(B * H)), dim3(256), 0, stream,
                       lg, vT, g, go, (int)S, (int)N, Np8, (int)H);
  }
  if ((rc = check_launch("f32_pwa_average"))) return rc;
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, go, w_o, nullptr, nullptr, m, out, M, hc, (int)c_m,
                  stream, "f32_pwa_out");
}

// ---------------------------------------------------------------------------
// PairMixer trunk glue, fp32 arithmetic (a trunk run with autocast off).
//   bioemu_ln_linear_fwd_f32   out = (base +) LN(x) W^T over M rows: the recycling
//                              updates s = s_init + s_recycle(s_norm(s)) and
//                              z = z_init + z_recycle(z_norm(z)) (pairmixer.py:276-283)
//   bioemu_trunk_uncond_fwd_f32  z_init + uncond_transition(z_norm(z_init)) (:266-273)
//   bioemu_distogram_fwd_f32   (z + z^T) W^T + b (embedders.py:191-206)
// ---------------------------------------------------------------------------
namespace bioemu {
namespace {

// sym[b, i, j, :] = z[b, i, j, :] + z[b, j, i, :]; one thread per 4 channels.
__global__ __launch_bounds__(256) void symmetrize_f32_kernel(const float* __restrict__ z, float* __restrict__ sym,
                                                             int N, int C, long long quads) {
  const long long q = (long long)blockIdx.x * 256 + threadIdx.x;
  if (q >= quads) return;
  const int cq = C / 4;
  const long long pair = q / cq;
  const int c = (int)(q % cq) * 4;
  const long long b = pair / ((long long)N * N), r = pair % ((long long)N * N);
  const int i = (int)(r / N), j = (int)(r % N);
  const f32x4 a = *reinterpret_cast<const f32x4*>(z + (size_t)pair * C + c);
  const f32x4 t = *reinterpret_cast<const f32x4*>(z + (((size_t)b * N + j) * N + i) * C + c);
  *reinterpret_cast<f32x4*>(sym + (size_t)pair * C + c) = a + t;
}

}  // namespace
}  // namespace bioemu

extern "C" size_t bioemu_ln_linear_f32_workspace_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return (size_t)round_up(M * K * 4, 256);
}

extern "C" int bioemu_ln_linear_fwd_f32(const float* x, const float* norm_w, const float* norm_b, const float* w,
                                        const float* base, float* out, void* workspace, size_t workspace_bytes,
                                        int64_t M, int64_t K, int64_t N, hipStream_t stream) {
  if (M <= 0 || K <= 0 || K % 8 || N <= 0 || N % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "ln_linear_f32: in dim a multiple of 8, out dim of 32 (got %lld, %lld)",
                     (long long)K, (long long)N);
  if (!x || !norm_w || !w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "ln_linear_f32: null pointer argument");
  if (!aligned16(x) || !aligned16(w) || !aligned16(out) || !aligned16(workspace) || (base && !aligned16(base)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "ln_linear_f32: tensors must be 16-byte aligned");
  if (workspace_bytes < bioemu_ln_linear_f32_workspace_bytes(M, K))
    return set_error(BIOEMU_ERR_WORKSPACE, "ln_linear_f32: workspace too small");
  float* xn = static_cast<float*>(workspace);
  const int rc = rows_ln_f32(x, norm_w, norm_b, xn, M, (int)K, stream, "f32_ln_linear_layernorm");
  if (rc) return rc;
  return gemm_f32(base ? kGemmEpiResidual : kGemmEpiStore, xn, w, nullptr, nullptr, base, out, M, (int)K, (int)N,
                  stream, "f32_ln_linear");
}

extern "C" size_t bioemu_trunk_uncond_f32_workspace_bytes(int64_t P, int64_t Dc, int64_t hidden) {
  if (P <= 0 || Dc <= 0 || hidden <= 0) return 0;
  return (size_t)round_up(P * Dc * 4, 256) + bioemu_transition_f32_workspace_bytes(P, Dc, hidden);
}

extern "C" int bioemu_trunk_uncond_fwd_f32(const float* z_init, const float* z_norm_w, const float* z_norm_b,
                                           const float* t_norm_w, const float* t_norm_b, const float* fc1_w,
                                           const float* fc2_w, const float* fc3_w, float* out, void* workspace,
                                           size_t workspace_bytes, int64_t P, int64_t Dc, int64_t hidden,
                                           hipStream_t stream) {
  if (P <= 0 || Dc <= 0 || Dc % 32 || hidden <= 0 || hidden % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "trunk_uncond_f32: dim and hidden must be multiples of 32 (got %lld, %lld)",
                     (long long)Dc, (long long)hidden);
  if (!z_init || !z_norm_w || !t_norm_w || !fc1_w || !fc2_w || !fc3_w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond_f32: null pointer argument");
  if (!aligned16(z_init) || !aligned16(out) || !aligned16(fc1_w) || !aligned16(fc2_w) || !aligned16(fc3_w) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond_f32: tensors must be 16-byte aligned");
  if (workspace_bytes < bioemu_trunk_uncond_f32_workspace_bytes(P, Dc, hidden))
    return set_error(BIOEMU_ERR_WORKSPACE, "trunk_uncond_f32: workspace too small");
  float* zn = static_cast<float*>(workspace);
  void* tws = static_cast<char*>(workspace) + round_up(P * Dc * 4, 256);
  const int rc = rows_ln_f32(z_init, z_norm_w, z_norm_b, zn, P, (int)Dc, stream, "f32_trunk_z_norm");
  if (rc) return rc;
  return transition_f32_res(zn, z_init, t_norm_w, t_norm_b, fc1_w, fc2_w, fc3_w, out, tws, P, Dc, hidden, Dc, 1, 1,
                            stream);
}

extern "C" size_t bioemu_distogram_f32_workspace_bytes(int64_t B, int64_t N, int64_t c_z) {
  if (B <= 0 || N <= 0 || c_z <= 0) return 0;
  return (size_t)round_up(B * N * N * c_z * 4, 256);
}

extern "C" int bioemu_distogram_fwd_f32(const float* z, const float* w, const float* b, float* out, void* workspace,
                                        size_t workspace_bytes, int64_t B, int64_t N, int64_t c_z, int64_t num_bins,
                                        hipStream_t stream) {
  if (c_z <= 0 || c_z % 8 || num_bins <= 0 || num_bins % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "distogram_f32: c_z a multiple of 8, num_bins of 32 (got %lld, %lld)",
                     (long long)c_z, (long long)num_bins);
  if (B <= 0 || N <= 0) return set_error(BIOEMU_ERR_INVALID_ARG, "distogram_f32: bad shape B=%lld N=%lld",
                                         (long long)B, (long long)N);
  if (!z || !w || !b || !out || !workspace) return set_error(BIOEMU_ERR_INVALID_ARG, "distogram_f32: null pointer");
  if (!aligned16(z) || !aligned16(w) || !aligned16(out) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "distogram_f32: tensors must be 16-byte aligned");
  if (workspace_bytes < bioemu_distogram_f32_workspace_bytes(B, N, c_z))
    return set_error(BIOEMU_ERR_WORKSPACE, "distogram_f32: workspace too small");
  float* sym = static_cast<float*>(workspace);
  const long long quads = B * N * N * c_z / 4;
  {
    KernelTimerScope timed("f32_symmetrize", stream);
    hipLaunchKernelGGL(symmetrize_f32_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, z, sym,
                       (int)N, (int)c_z, quads);
  }
  const int rc = check_launch("f32_symmetrize");
  if (rc) return rc;
  return gemm_f32(kGemmEpiStore, sym, w, nullptr, b, nullptr, out, B * N * N, (int)c_z, (int)num_bins, stream,
                  "f32_distogram");
}

// ---------------------------------------------------------------------------
// Triangle attention in fp32 (AlphaFold3 suppl. Alg. 14/15 with the masking
// of the reference's attention: a masked key's logit is replaced by -1e6).
// Starting node: sequence (b, i) is the pair row z[b, i, :]; its queries and
// keys are j, k along that row, bias[b][h][j][k] = LN(z[b, j, k]) . w_b[h]
// (shared by every row i of batch b), key mask mask[b, i, k].  The ending node
// runs the same on z^T and mask^T and transposes the gated attention output
// back before the output projection, so its residual rows are z's own.
// ---------------------------------------------------------------------------
namespace bioemu {
namespace {

// dst[b][i][j][:] = src[b][j][i][:] for C fp32 channels (C % 4 == 0): one
// thread per 16-byte chunk, consecutive threads along a destination row.
__global__ __launch_bounds__(256) void transpose_pairs_f32_kernel(const float* __restrict__ src,
                                                                  float* __restrict__ dst, int N, int C,
                                                                  long long total) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int cq = C / 4;
  const long long pair = t / cq;
  const int q = (int)(t - pair * cq);
  const long long nn = (long long)N * N;
  const long long b = pair / nn, r = pair - b * nn;
  const long long i = r / N, j = r - i * N;
  const f32x4 v = *reinterpret_cast<const f32x4*>(src + ((b * N + j) * N + i) * C + 4 * q);
  *reinterpret_cast<f32x4*>(dst + pair * C + 4 * q) = v;
}

// dst[b][i][j] = src[b][j][i] over B x N x N bytes.
__global__ __launch_bounds__(256) void transpose_mask_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                             int N, long long total) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const long long nn = (long long)N * N;
  const long long b = t / nn, r = t - b * nn;
  const long long i = r / N, j = r - i * N;
  dst[t] = src[(b * N + j) * N + i];
}

int transpose_pairs_f32(const float* src, float* dst, long long B, int N, int C, hipStream_t stream,
                        const char* name) {
  const long long total = B * N * N * (C / 4);
  KernelTimerScope timed(name, stream);
  hipLaunchKernelGGL(transpose_pairs_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, src, dst,
                     N, C, total);
  return check_launch(name);
}

}  // namespace
}  // namespace bioemu

extern "C" size_t bioemu_triatt_f32_workspace_bytes(int64_t B, int64_t N, int64_t D, int64_t H) {
  if (B <= 0 || N <= 0 || D <= 0 || H <= 0) return 0;
  const int64_t P = B * N * N, ld = round_up(N, 32);
  return (size_t)round_up(P * D * 4, 256) + (size_t)round_up(P, 256) +
         attn_f32_layout(P, (int)D, B * N * D * ld, B * H * N * ld, true, nullptr, nullptr);
}

extern "C" int bioemu_triatt_fwd_f32(const float* z, const uint8_t* mask, const float* norm_w, const float* norm_b,
                                     const float* w_proj, const float* w_o, float* out, void* workspace,
                                     size_t workspace_bytes, int64_t B, int64_t N, int64_t D, int64_t H, int starting,
                                     int residual, hipStream_t stream) {
  if (H <= 0 || D % H || D / H != 32 || (D != 32 && D != 128))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "triatt_f32: supported are c = 32 or 128 with heads of 32 channels (got c=%lld H=%lld)",
                     (long long)D, (long long)H);
  if (B <= 0 || N <= 0 || B * N > 65535)
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt_f32: bad shape B=%lld N=%lld (B * N <= 65535)", (long long)B,
                     (long long)N);
  if (!z || !mask || !norm_w || !norm_b || !w_proj || !w_o || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt_f32: null pointer argument");
  if (!aligned16(z) || !aligned16(out) || !aligned16(w_proj) || !aligned16(w_o) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt_f32: tensors must be 16-byte aligned");
  if (out == z && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt_f32: out may alias z only with residual=1");
  if (workspace_bytes < bioemu_triatt_f32_workspace_bytes(B, N, D, H))
    return set_error(BIOEMU_ERR_WORKSPACE, "triatt_f32: workspace too small");
  const long long P = B * N * N;
  const int ld = (int)round_up(N, 32), c = (int)D;
  char* p = static_cast<char*>(workspace);
  float* zt = reinterpret_cast<float*>(p);
  p += round_up(P * D * 4, 256);
  uint8_t* mt = reinterpret_cast<uint8_t*>(p);
  p += round_up(P, 256);
  AttnF32Buffers buf;
  attn_f32_layout(P, c, B * N * D * ld, B * H * N * ld, true, &buf, p);
  const float* src = z;
  const uint8_t* msk = mask;
  int rc = 0;
  if (!starting) {
    if ((rc = transpose_pairs_f32(z, zt, B, (int)N, c, stream, "f32_triatt_transpose_in"))) return rc;
    {
      KernelTimerScope timed("f32_triatt_transpose_mask", stream);
      hipLaunchKernelGGL(transpose_mask_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, stream, mask, mt,
                         (int)N, P);
    }
    if ((rc = check_launch("f32_triatt_transpose_mask"))) return rc;
    src = zt;
    msk = mt;
  }
  // w_proj rows: [Wq; Wk; Wv] (3c), Wg (c), Wb (H)
  rc = attn_f32_projections(src, norm_w, norm_b, w_proj, nullptr, w_proj + 3 * D * D, buf, P, c, (int)N, ld, stream);
  if (rc) return rc;
  rc = pair_proj_f32(src, norm_w, norm_b, w_proj + 4 * D * D, buf.bias, P, (int)N, (int)N, ld, (int)H, c, stream,
                     "f32_triatt_bias");
  if (rc) return rc;
  {
    KernelTimerScope timed("f32_triatt_attention", stream);
    const dim3 grid((unsigned)((N + 127) / 128), (unsigned)H, (unsigned)(B * N));
    hipLaunchKernelGGL(attn_f32_kernel<32>, grid, dim3(256), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, msk,
                       buf.go, (int)N, ld, (int)H, c, (int)N, 1.0f / std::sqrt(32.0f), 1);
  }
  if ((rc = check_launch("f32_triatt_attention"))) return rc;
  const float* go = buf.go;
  if (!starting) {
    if ((rc = transpose_pairs_f32(buf.go, zt, B, (int)N, c, stream, "f32_triatt_transpose_out"))) return rc;
    go = zt;
  }
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, go, w_o, nullptr, nullptr, z, out, P, c, c, stream,
                  "f32_triatt_proj_o");
}
