// fp32 arithmetic path of the denoiser's ops, for gfx950.
//
// The reference runs its denoiser with autocast off (src/bioemu2/biomoa/models/
// score_model.py:355, model.py:387), so its attention-with-pair-bias
// (attention_pair_bias.py:128-225), sliding-window attention (:277-340) and
// token transitions (transition.py:52-91) compute in fp32 on fp32 inputs.  These
// entry points do the same: fp32 operands and fp32 accumulation throughout.
//
//   gemm_f32      out = epi(A W^T) on v_mfma_f32_32x32x2_f32.  A wave owns a
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
//                 g: one thread per query, 64-key blocks of K and V in LDS,
//                 blockwise online softmax.
//   swa_attn_f32  the same over the sliding key window of each 32-atom window.
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmEpiStore = 0, kGemmEpiSigmoid = 1, kGemmEpiSwiGLU = 2, kGemmEpiResidual = 3;

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
                                                       const float* res, float* out, long long M, int K, int N) {
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

template <int CZ>
__global__ __launch_bounds__(256) void pair_proj_f32_kernel(const float* __restrict__ z, const float* __restrict__ g,
                                                            const float* __restrict__ b, const float* __restrict__ w,
                                                            float* __restrict__ out, long long P, long long inner,
                                                            int H) {
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
  const long long outer = p / inner, idx = p % inner;
  for (int hh = 0; hh < H; ++hh) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CZ; ++c) acc += w[hh * CZ + c] * v[c];
    out[((size_t)outer * H + hh) * inner + idx] = acc;
  }
}

// Full attention: grid (ceil(N / 128), H, B * mult); thread = query.
template <int D>
__global__ __launch_bounds__(128) void attn_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ g,
                                                       const float* __restrict__ bias,
                                                       const uint8_t* __restrict__ mask, float* __restrict__ go,
                                                       int N, int H, int c_s, int mult) {
  __shared__ float ks[64][D], vs[64][D];
  __shared__ uint8_t ms[64];
  const int hd = blockIdx.y, bm = blockIdx.z, b = bm / mult;
  const int i = blockIdx.x * 128 + threadIdx.x;
  const bool qvalid = i < N;
  const int ic = qvalid ? i : 0;
  float qv[D], o[D];
  const float* qr = q + ((size_t)bm * N + ic) * c_s + hd * D;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qv[d] = qr[d];
    o[d] = 0.f;
  }
  const float sqrt_d = sqrtf((float)D);
  const float* brow = bias + (((size_t)b * H + hd) * N + ic) * N;
  float m = -INFINITY, l = 0.f;
  for (int j0 = 0; j0 < N; j0 += 64) {
    __syncthreads();
    for (int t = threadIdx.x; t < 64 * D; t += 128) {
      const int kk = t / D, d = t % D, j = j0 + kk;
      const size_t off = ((size_t)bm * N + (j < N ? j : 0)) * c_s + hd * D + d;
      ks[kk][d] = j < N ? k[off] : 0.f;
      vs[kk][d] = j < N ? v[off] : 0.f;
    }
    if (threadIdx.x < 64) ms[threadIdx.x] = j0 + threadIdx.x < N ? mask[(size_t)b * N + j0 + threadIdx.x] : 0;
    __syncthreads();
    const int jn = min(64, N - j0);
    float lg[64];
    float bmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) {
      if (jj < jn) {
        float dot = 0.f;
#pragma unroll
        for (int d = 0; d < D; ++d) dot += qv[d] * ks[jj][d];
        const float x = ms[jj] ? dot / sqrt_d + brow[j0 + jj] : -1e6f;
        lg[jj] = x;
        bmax = fmaxf(bmax, x);
      }
    }
    const float m_new = fmaxf(m, bmax);
    const float alpha = __expf(m - m_new);
    l *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] *= alpha;
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) {
      if (jj < jn) {
        const float p = __expf(lg[jj] - m_new);
        l += p;
#pragma unroll
        for (int d = 0; d < D; ++d) o[d] += p * vs[jj][d];
      }
    }
    m = m_new;
  }
  if (!qvalid) return;
  const size_t off = ((size_t)bm * N + i) * c_s + hd * D;
  const float inv = 1.0f / l;
#pragma unroll
  for (int d = 0; d < D; ++d) go[off + d] = g[off + d] * (o[d] * inv);
}

// Sliding-window attention: grid (NW, ceil(heads / 4), B * mult); thread = (head in group, query in window).
template <int D>
__global__ __launch_bounds__(128) void swa_attn_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, const float* __restrict__ g,
                                                           const float* __restrict__ bias,
                                                           const uint8_t* __restrict__ mask, float* __restrict__ go,
                                                           int NW, int Hk, int heads, int c_s, int mult) {
  constexpr int W = 32;
  __shared__ float ks[4][W][D], vs[4][W][D];
  __shared__ uint8_t ms[W];
  const int w = blockIdx.x, bm = blockIdx.z, b = bm / mult;
  const int hq = threadIdx.x / W, iq = threadIdx.x % W;
  const int hd = blockIdx.y * 4 + hq;
  const bool hvalid = hd < heads;
  const int hc = hvalid ? hd : 0;
  const int NA = NW * W, ctx = (Hk - W) / 2;
  const int aq = w * W + iq;
  float qv[D], o[D];
  const float* qr = q + ((size_t)bm * NA + aq) * c_s + hc * D;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qv[d] = qr[d];
    o[d] = 0.f;
  }
  const float sqrt_d = sqrtf((float)D);
  const float* brow = bias + ((((size_t)b * NW + w) * heads + hc) * W + iq) * Hk;
  float m = -INFINITY, l = 0.f;
  for (int t0 = 0; t0 < Hk; t0 += W) {
    __syncthreads();
    for (int t = threadIdx.x; t < 4 * W * D; t += 128) {
      const int gh = t / (W * D), kk = (t / D) % W, d = t % D;
      const int a = w * W - ctx + t0 + kk, hh = blockIdx.y * 4 + gh;
      const bool ok = a >= 0 && a < NA && hh < heads;
      const size_t off = ((size_t)bm * NA + (ok ? a : 0)) * c_s + (hh < heads ? hh : 0) * D + d;
      ks[gh][kk][d] = ok ? k[off] : 0.f;
      vs[gh][kk][d] = ok ? v[off] : 0.f;
    }
    if (threadIdx.x < W) {
      const int a = w * W - ctx + t0 + threadIdx.x;
      ms[threadIdx.x] = (a >= 0 && a < NA) ? mask[(size_t)b * NA + a] : 0;
    }
    __syncthreads();
    float lg[W];
    float bmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < W; ++jj) {
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) dot += qv[d] * ks[hq][jj][d];
      const float x = ms[jj] ? dot / sqrt_d + brow[t0 + jj] : -1e6f;
      lg[jj] = x;
      bmax = fmaxf(bmax, x);
    }
    const float m_new = fmaxf(m, bmax);
    const float alpha = __expf(m - m_new);
    l *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] *= alpha;
#pragma unroll
    for (int jj = 0; jj < W; ++jj) {
      const float p = __expf(lg[jj] - m_new);
      l += p;
#pragma unroll
      for (int d = 0; d < D; ++d) o[d] += p * vs[hq][jj][d];
    }
    m = m_new;
  }
  if (!hvalid) return;
  const size_t off = ((size_t)bm * NA + aq) * c_s + hd * D;
  const float inv = 1.0f / l;
#pragma unroll
  for (int d = 0; d < D; ++d) go[off + d] = g[off + d] * (o[d] * inv);
}

int gemm_f32(int epi, const float* A, const float* W, const float* W2, const float* bias, const float* res, float* out,
             long long M, int K, int N, hipStream_t stream, const char* name) {
  if (K % 8 || N % 32 || M <= 0)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "%s: fp32 GEMM needs K %% 8 == 0 and N %% 32 == 0 (K=%d N=%d)", name, K,
                     N);
  const long long blocks = (M + 31) / 32 * (N / 32);
  const unsigned grid = (unsigned)((blocks + 3) / 4);
  KernelTimerScope timed(name, stream);
  switch (epi) {
    case kGemmEpiStore:
      hipLaunchKernelGGL(gemm_f32_kernel<kGemmEpiStore>, dim3(grid), dim3(256), 0, stream, A, W, W2, bias, res, out, M,
                         K, N);
      break;
    case kGemmEpiSigmoid:
      hipLaunchKernelGGL(gemm_f32_kernel<kGemmEpiSigmoid>, dim3(grid), dim3(256), 0, stream, A, W, W2, bias, res, out,
                         M, K, N);
      break;
    case kGemmEpiSwiGLU:
      hipLaunchKernelGGL(gemm_f32_kernel<kGemmEpiSwiGLU>, dim3(grid), dim3(256), 0, stream, A, W, W2, bias, res, out,
                         M, K, N);
      break;
    default:
      hipLaunchKernelGGL(gemm_f32_kernel<kGemmEpiResidual>, dim3(grid), dim3(256), 0, stream, A, W, W2, bias, res,
                         out, M, K, N);
      break;
  }
  return check_launch(name);
}

int rows_ln_f32(const float* x, const float* g, const float* b, float* y, long long rows, int K, hipStream_t stream,
                const char* name, const float* x2 = nullptr, int K2 = 0) {
  KernelTimerScope timed(name, stream);
  hipLaunchKernelGGL(rows_ln_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, K, x2, K2, g, b,
                     y, rows);
  return check_launch(name);
}

int pair_proj_f32(const float* z, const float* g, const float* b, const float* w, float* out, long long P,
                  long long inner, int H, int c_z, hipStream_t stream, const char* name) {
  const unsigned grid = (unsigned)((P + 255) / 256);
  KernelTimerScope timed(name, stream);
  if (c_z == 128)
    hipLaunchKernelGGL(pair_proj_f32_kernel<128>, dim3(grid), dim3(256), 0, stream, z, g, b, w, out, P, inner, H);
  else if (c_z == 32)
    hipLaunchKernelGGL(pair_proj_f32_kernel<32>, dim3(grid), dim3(256), 0, stream, z, g, b, w, out, P, inner, H);
  else if (c_z == 16)
    hipLaunchKernelGGL(pair_proj_f32_kernel<16>, dim3(grid), dim3(256), 0, stream, z, g, b, w, out, P, inner, H);
  else
    return set_error(BIOEMU_ERR_UNSUPPORTED, "%s: c_z %d unsupported (16, 32 or 128)", name, c_z);
  return check_launch(name);
}

// Token-side projections shared by both attentions: optional LN, then q (+ q bias), k, v, sigmoid(g).
struct AttnF32Buffers {
  float *sn, *q, *k, *v, *g, *go, *bias;
};

size_t attn_f32_layout(long long rows, int c_s, long long bias_elems, bool norm, AttnF32Buffers* buf, char* base) {
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
  take(&b->v, (size_t)rows * c_s);
  take(&b->g, (size_t)rows * c_s);
  take(&b->go, (size_t)rows * c_s);
  take(&b->bias, (size_t)bias_elems);
  return off;
}

int attn_f32_projections(const float* s, const float* norm_s_w, const float* norm_s_b, const float* w_qkv,
                         const float* q_bias, const float* w_g, AttnF32Buffers& buf, long long rows, int c_s,
                         hipStream_t stream) {
  const float* src = s;
  int rc = 0;
  if (norm_s_w) {
    rc = rows_ln_f32(s, norm_s_w, norm_s_b, buf.sn, rows, c_s, stream, "f32_layernorm");
    src = buf.sn;
  }
  const size_t cc = (size_t)c_s * c_s;
  if (!rc) rc = gemm_f32(kGemmEpiStore, src, w_qkv, nullptr, q_bias, nullptr, buf.q, rows, c_s, c_s, stream, "f32_proj_q");
  if (!rc)
    rc = gemm_f32(kGemmEpiStore, src, w_qkv + cc, nullptr, nullptr, nullptr, buf.k, rows, c_s, c_s, stream, "f32_proj_k");
  if (!rc)
    rc = gemm_f32(kGemmEpiStore, src, w_qkv + 2 * cc, nullptr, nullptr, nullptr, buf.v, rows, c_s, c_s, stream,
                  "f32_proj_v");
  if (!rc) rc = gemm_f32(kGemmEpiSigmoid, src, w_g, nullptr, nullptr, nullptr, buf.g, rows, c_s, c_s, stream, "f32_proj_g");
  return rc;
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_apb_f32_workspace_bytes(int64_t B, int64_t mult, int64_t N, int64_t c_s, int64_t H) {
  if (B <= 0 || mult <= 0 || N <= 0 || c_s <= 0 || H <= 0) return 0;
  return attn_f32_layout(B * mult * N, (int)c_s, B * H * N * N, true, nullptr, nullptr);
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
  attn_f32_layout(rows, (int)c_s, B * H * N * N, true, &buf, static_cast<char*>(workspace));
  int rc = attn_f32_projections(s, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, buf, rows, (int)c_s, stream);
  if (rc) return rc;
  rc = pair_proj_f32(z, norm_z_w, norm_z_b, w_z, buf.bias, B * N * N, N * N, (int)H, (int)c_z, stream,
                     "f32_pair_bias");
  if (rc) return rc;
  {
    KernelTimerScope timed("f32_attention", stream);
    const dim3 grid((unsigned)((N + 127) / 128), (unsigned)H, (unsigned)(B * mult));
    if (c_s / H == 24)
      hipLaunchKernelGGL(attn_f32_kernel<24>, grid, dim3(128), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, mask,
                         buf.go, (int)N, (int)H, (int)c_s, (int)mult);
    else
      hipLaunchKernelGGL(attn_f32_kernel<32>, grid, dim3(128), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, mask,
                         buf.go, (int)N, (int)H, (int)c_s, (int)mult);
  }
  rc = check_launch("f32_attention");
  if (rc) return rc;
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, buf.go, w_o, nullptr, nullptr, s, out, rows, (int)c_s,
                  (int)c_s, stream, "f32_proj_o");
}

extern "C" size_t bioemu_swa_f32_workspace_bytes(int64_t B, int64_t mult, int64_t NW, int64_t W, int64_t H,
                                                 int64_t c_s, int64_t heads) {
  if (B <= 0 || mult <= 0 || NW <= 0 || W != 32 || H <= 0 || c_s <= 0 || heads <= 0) return 0;
  return attn_f32_layout(B * mult * NW * W, (int)c_s, B * NW * heads * W * H, true, nullptr, nullptr);
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
  if (out == s && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa_f32: out may alias s only with residual=1");
  if (workspace_bytes < bioemu_swa_f32_workspace_bytes(B, mult, NW, W, H, c_s, heads))
    return set_error(BIOEMU_ERR_WORKSPACE, "swa_f32: workspace too small");
  const long long rows = B * mult * NW * W;
  AttnF32Buffers buf;
  attn_f32_layout(rows, (int)c_s, B * NW * heads * W * H, true, &buf, static_cast<char*>(workspace));
  int rc = attn_f32_projections(s, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, buf, rows, (int)c_s, stream);
  if (rc) return rc;
  rc = pair_proj_f32(z, norm_z_w, norm_z_b, w_z, buf.bias, B * NW * W * H, W * H, (int)heads, (int)c_z, stream,
                     "f32_swa_pair_bias");
  if (rc) return rc;
  {
    KernelTimerScope timed("f32_swa_attention", stream);
    hipLaunchKernelGGL(swa_attn_f32_kernel<32>, dim3((unsigned)NW, (unsigned)((heads + 3) / 4), (unsigned)(B * mult)),
                       dim3(128), 0, stream, buf.q, buf.k, buf.v, buf.g, buf.bias, mask, buf.go, (int)NW, (int)H,
                       (int)heads, (int)c_s, (int)mult);
  }
  rc = check_launch("f32_swa_attention");
  if (rc) return rc;
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, buf.go, w_o, nullptr, nullptr, s, out, rows, (int)c_s,
                  (int)c_s, stream, "f32_proj_o");
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
  return gemm_f32(residual ? kGemmEpiResidual : kGemmEpiStore, hbuf, fc3_w, nullptr, nullptr, x, out, M, (int)hidden,
                  (int)out_dim, stream, "f32_transition_out");
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
