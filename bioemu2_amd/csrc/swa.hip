// Sliding-window attention with pair bias (the denoiser's atom transformer)
// for gfx950.
//
// Reference: AttentionPairBiasSlidingWindow.forward
// (src/bioemu2/biomoa/ops/attention_pair_bias.py:277-340):
//   s' = LN_s(s) if initial_norm;  q = s' Wq^T + q_bias;  k, v = s' Wk^T, s' Wv^T
//   g = sigmoid(s' Wg^T);  each window of W = 32 queries attends to the H keys
//   centred on it: atom positions [w W - ctx, w W - ctx + H), ctx = (H - W) / 2,
//   zero k / v and a False mask outside the sequence (:302-317);
//   A = q k^T / sqrt(d) + bias[b, w, h] (bias = (LN_z(z) Wz^T) per (b, window),
//   shared by the M copies, :319-330);  A[..., ~mask_key] = -1e6 (replace);
//   out = (g * softmax(A) v) Wo^T   (+ s when residual != 0).
// s is [B*M*NW, W, c_s]: row (b, m, w, i) = atom w W + i of copy (b, m), so
// each (b, m) is one contiguous [NA = NW W][c_s] sequence.
//
// Kernels: token LN / GEMMs for the per-atom projections (token.hip; v is
// written transposed, [c_s][NA] per copy); swa_pair_bias reads z once and
// writes a bf16 [B][NW][heads][W][H] bias (the M copies re-read it from L2);
// swa_attn runs one wave per (copy, window, head): S^T = K Q^T over 32-key
// blocks (key rows in perm32 order so every lane holds 16 consecutive keys),
// bias + mask + online softmax in registers, O^T = V^T P^T with P straight
// from the registers, and writes g * o.
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int DH = 32;   // head dim
constexpr int WQ = 32;   // queries per window
constexpr int kMaxHeads = 12;   // c_s = 32 heads in {64, 128, 384}

// ---------------------------------------------------------------------------
// bias[b][w][h][i][j] = log2(e) * LN_z(z[b][w][i][j]) . Wz[h]; one thread per pair
// (consecutive lanes = consecutive keys: coalesced 32-byte reads, and each
// head's 2-byte stores of a wave form one 128-byte run).
// ---------------------------------------------------------------------------
template <int CZ, int HEADS>
__global__ __launch_bounds__(256) void swa_bias_kernel(const bf16* __restrict__ z, const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, const bf16* __restrict__ wz,
                                                       bf16* __restrict__ bias, long long pairs, int HK) {
  __shared__ float wl[HEADS * CZ];
  __shared__ float gl[CZ], bl[CZ];
  for (int t = threadIdx.x; t < HEADS * CZ; t += blockDim.x) wl[t] = bf2f(wz[t]);
  for (int t = threadIdx.x; t < CZ; t += blockDim.x) {
    gl[t] = gamma[t];
    bl[t] = beta ? beta[t] : 0.f;
  }
  __syncthreads();
  const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // (b, w, i, j)
  if (r >= pairs) return;
  const int j = (int)(r % HK);
  const long long row = r / HK;                   // (b, w, i)
  const int i = (int)(row % WQ);
  const long long bw = row / WQ;                  // b * NW + w
  float v[CZ];
#pragma unroll
  for (int c = 0; c < CZ; c += 8) unpack8(load8(z + (size_t)r * CZ + c), v + c);
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CZ; ++c) sum += v[c];
  const float mean = sum * (1.0f / CZ);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CZ; ++c) {
    const float d = v[c] - mean;
    ss += d * d;
  }
  const float rstd = rsqrtf(ss * (1.0f / CZ) + 1e-5f);
#pragma unroll
  for (int c = 0; c < CZ; ++c) v[c] = (v[c] - mean) * rstd * gl[c] + bl[c];
#pragma unroll
  for (int h = 0; h < HEADS; ++h) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CZ; ++c) acc += v[c] * wl[h * CZ + c];
    bias[(((size_t)bw * HEADS + h) * WQ + i) * HK + j] = f2bf(acc * kLog2e);   // log2 units (base-2 softmax)
  }
}

template <int CZ, int HEADS>
void launch_swa_bias(const bf16* z, const float* gamma, const float* beta, const bf16* wz, bf16* bias,
                     long long pairs, int HK, hipStream_t stream) {
  hipLaunchKernelGGL((swa_bias_kernel<CZ, HEADS>), dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, stream, z,
                     gamma, beta, wz, bias, pairs, HK);
}

template <int CZ>
void launch_swa_bias(int heads, const bf16* z, const float* gamma, const float* beta, const bf16* wz, bf16* bias,
                     long long pairs, int HK, hipStream_t stream) {
  if (heads == 2) launch_swa_bias<CZ, 2>(z, gamma, beta, wz, bias, pairs, HK, stream);
  else if (heads == 4) launch_swa_bias<CZ, 4>(z, gamma, beta, wz, bias, pairs, HK, stream);
  else launch_swa_bias<CZ, 12>(z, gamma, beta, wz, bias, pairs, HK, stream);
}

// ---------------------------------------------------------------------------
// Attention.  Block = (window w, 4 heads, copy bm); wave -> head 4 blockIdx.y + wave.
// q arrives pre-scaled by log2(e)/sqrt(d) and the bias in log2 units, so
// q.k + bias is the logit in base 2.  Per window key j (atom kstart + j) the
// workgroup keeps in LDS kv[j] = 1, c0[j] = 0 for a valid key and kv = 0,
// c0 = -1e6 log2(e) for a masked one or one outside the sequence (the
// reference's replacement): x = kv (q.k + bias) + c0.  Key blocks are read
// kChunk at a time, every operand of a chunk requested before its first use;
// addresses of keys outside the sequence are clamped to atom 0 (their logit is
// replaced, and their V is selected as zero, so the values read do not matter).
// ---------------------------------------------------------------------------
constexpr int kChunk = 2;   // 32-key blocks whose operands are fetched together

__global__ __launch_bounds__(256) void swa_attn_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                       const bf16* __restrict__ vt, const bf16* __restrict__ g,
                                                       const bf16* __restrict__ bias,
                                                       const uint8_t* __restrict__ mask, bf16* __restrict__ go,
                                                       int NW, int HK, int heads, int mult) {
  extern __shared__ __attribute__((aligned(16))) float key_terms[];   // kv[HK] then c0[HK]
  float* kvl = key_terms;
  float* c0l = key_terms + HK;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, hh = lane >> 5;
  const int w = blockIdx.x, bm = blockIdx.z, b = bm / mult;
  const int NA = NW * WQ;
  const int kstart = w * WQ - (HK - WQ) / 2;
  const float masked_logit = -1e6f * kLog2e;
  for (int j = threadIdx.x; j < HK; j += blockDim.x) {
    const int kp = kstart + j;
    const bool valid = kp >= 0 && kp < NA && mask[(size_t)b * NA + kp] != 0;
    kvl[j] = valid ? 1.f : 0.f;
    c0l[j] = valid ? 0.f : masked_logit;
  }
  __syncthreads();
  const int hd = blockIdx.y * 4 + wave;
  if (hd >= heads) return;   // after the only barrier
  const int CS = heads * DH;

  bf16x8 zero8;
#pragma unroll
  for (int t = 0; t < 8; ++t) zero8[t] = f2bf(0.f);

  const bf16* qrow = q + ((size_t)bm * NA + w * WQ + n) * CS + hd * DH;
  const bf16x8 qf0 = load8(qrow + 8 * hh);
  const bf16x8 qf1 = load8(qrow + 16 + 8 * hh);
  const bf16* kbase = k + (size_t)bm * NA * CS + hd * DH;
  const bf16* vbase = vt + ((size_t)bm * CS + hd * DH + perm32(n)) * NA;
  const bf16* brow = bias + ((((size_t)b * NW + w) * heads + hd) * WQ + n) * HK;

  f32x16 o = zero16();
  float m = -INFINITY, l = 0.f;
  for (int kc = 0; kc < HK; kc += 32 * kChunk) {
    // operands of the chunk's blocks (a block past HK repeats the last one and is skipped)
    bf16x8 kf[kChunk][2], vf[kChunk][2], bf[kChunk][2];
    bool run_in[kChunk];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int kb = min(kc + 32 * c, HK - 32);
      const int krow = kstart + kb + perm32(n);
      const bf16* kr = kbase + (size_t)(krow >= 0 && krow < NA ? krow : 0) * CS;
      kf[c][0] = load8(kr + 8 * hh);
      kf[c][1] = load8(kr + 16 + 8 * hh);
      // this lane's 16 keys are one run of atoms, entirely inside or outside the sequence
      const int kp = kstart + kb + 16 * hh;
      run_in[c] = kp >= 0 && kp < NA;
      const bf16* vp = vbase + (run_in[c] ? kp : 0);
      vf[c][0] = load8(vp);
      vf[c][1] = load8(vp + 8);
      bf[c][0] = load8(brow + kb + 16 * hh);
      bf[c][1] = load8(brow + kb + 16 * hh + 8);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int kb = kc + 32 * c;
      if (kb >= HK) break;   // uniform
      // S^T: lane (n, hh) register u <-> window key kb + 16 hh + u of query n
      f32x16 s = zero16();
      s = mfma32(kf[c][0], qf0, s);
      s = mfma32(kf[c][1], qf1, s);
      const float4* kv4 = reinterpret_cast<const float4*>(kvl + kb + 16 * hh);
      const float4* c04 = reinterpret_cast<const float4*>(c0l + kb + 16 * hh);
      float kv[16], c0[16];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float4 a = kv4[e], cc = c04[e];
        kv[4 * e] = a.x, kv[4 * e + 1] = a.y, kv[4 * e + 2] = a.z, kv[4 * e + 3] = a.w;
        c0[4 * e] = cc.x, c0[4 * e + 1] = cc.y, c0[4 * e + 2] = cc.z, c0[4 * e + 3] = cc.w;
      }
      float t[16];
      float bmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float x = __builtin_fmaf(s[u] + bf2f(u < 8 ? bf[c][0][u] : bf[c][1][u - 8]), kv[u], c0[u]);
        t[u] = x;
        bmax = fmaxf(bmax, x);
      }
      bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
      const float m_new = fmaxf(m, bmax);
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      float psum = 0.f;
      bf16x8 pb[2];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float p = fast_exp2(t[u] - m_new);
        psum += p;
        pb[u >> 3][u & 7] = f2bf(p);
      }
      l = l * alpha + psum;
#pragma unroll
      for (int u = 0; u < 16; ++u) o[u] *= alpha;
      // O^T += V^T P^T: lane (d slot, hh) supplies v^T[d][kp .. kp + 15] (zero outside)
      o = mfma32(run_in[c] ? vf[c][0] : zero8, pb[0], o);
      o = mfma32(run_in[c] ? vf[c][1] : zero8, pb[1], o);
    }
  }

  // D lane (n, hh) register u <-> channel 16 hh + u of query n
  const float inv = 1.0f / (l + __shfl_xor(l, 32));
  const size_t off = ((size_t)bm * NA + w * WQ + n) * CS + hd * DH + 16 * hh;
  const bf16x8 g0 = load8(g + off), g1 = load8(g + off + 8);
  float v[16];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    v[u] = bf2f(g0[u]) * (o[u] * inv);
    v[8 + u] = bf2f(g1[u]) * (o[8 + u] * inv);
  }
  store16(go + off, v);
}

struct SwaBuffers {
  bf16 *sn, *q, *k, *vt, *g, *go, *bias;
};

size_t swa_layout(int64_t B, int64_t BM, int64_t NW, int64_t HK, int64_t CS, int64_t heads, SwaBuffers* buf,
                  char* base) {
  const size_t tok = round_up(BM * NW * WQ * CS * 2, 256);
  const size_t bias_bytes = round_up((size_t)B * NW * heads * WQ * HK * 2, 256);
  if (buf) {
    bf16** slots[6] = {&buf->sn, &buf->q, &buf->k, &buf->vt, &buf->g, &buf->go};
    for (int t = 0; t < 6; ++t) *slots[t] = reinterpret_cast<bf16*>(base + t * tok);
    buf->bias = reinterpret_cast<bf16*>(base + 6 * tok);
  }
  return 6 * tok + bias_bytes;
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_swa_workspace_bytes(int64_t B, int64_t mult, int64_t NW, int64_t W, int64_t H,
                                             int64_t c_s, int64_t heads) {
  if (B <= 0 || mult <= 0 || NW <= 0 || W != WQ || H <= 0 || c_s <= 0 || heads <= 0) return 0;
  return swa_layout(B, B * mult, NW, H, c_s, heads, nullptr, nullptr);
}

extern "C" int bioemu_swa_fwd(const void* s, const void* z, const uint8_t* mask, const float* norm_s_w,
                              const float* norm_s_b, const void* w_qkv, const float* q_bias, const void* w_g,
                              const float* norm_z_w, const float* norm_z_b, const void* w_z, const void* w_o,
                              void* out, void* workspace, size_t workspace_bytes, int64_t B, int64_t mult,
                              int64_t NW, int64_t W, int64_t H, int64_t c_s, int64_t c_z, int64_t heads,
                              int residual, hipStream_t stream) {
  if (W != WQ || H < WQ || H > 16384 || H % 32 || (H - W) % 32 || heads <= 0 || heads > kMaxHeads || c_s != heads * DH ||
      (heads != 2 && heads != 4 && heads != 12) || (c_z != 16 && c_z != 32))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "swa: supported shapes are W=32, H <= 16384 a multiple of 32 with H-W a multiple of 32, head dim 32 "
                     "with c_s in {64, 128, 384}, c_z in {16, 32} (got W=%lld H=%lld c_s=%lld heads=%lld c_z=%lld)",
                     (long long)W, (long long)H, (long long)c_s, (long long)heads, (long long)c_z);
  if (B <= 0 || mult <= 0 || NW <= 0 || B * mult > 65535 || NW > 65535 || NW * WQ * c_s > (1LL << 30))
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa: bad shape B=%lld M=%lld NW=%lld", (long long)B, (long long)mult,
                     (long long)NW);
  if (!s || !z || !mask || !w_qkv || !q_bias || !w_g || !norm_z_w || !w_z || !w_o || !out || !workspace ||
      (norm_s_w == nullptr) != (norm_s_b == nullptr))
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa: null pointer argument");
  if (!aligned16(s) || !aligned16(z) || !aligned16(mask) || !aligned16(out) || !aligned16(w_qkv) ||
      !aligned16(w_g) || !aligned16(w_o) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa: tensors must be 16-byte aligned");
  if (out == s && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "swa: out may alias s only with residual=1");
  const int64_t BM = B * mult;
  if (workspace_bytes < swa_layout(B, BM, NW, H, c_s, heads, nullptr, nullptr))
    return set_error(BIOEMU_ERR_WORKSPACE, "swa: workspace too small");
  SwaBuffers buf;
  swa_layout(B, BM, NW, H, c_s, heads, &buf, static_cast<char*>(workspace));
  const int64_t NA = NW * WQ;
  const int64_t M = BM * NA;
  const bf16* wqkv = static_cast<const bf16*>(w_qkv);

  // Every copy is one [NA][c_s] sequence (NA is a multiple of 32: no row padding), so
  // without initial_norm the projections read s itself.
  int rc = 0;
  const void* sn = s;
  if (norm_s_w) {
    rc = token_layernorm(s, norm_s_w, norm_s_b, buf.sn, BM, NA, NA, c_s, stream);
    sn = buf.sn;
  }
  // q carries the attention's softmax scale in base 2 (swa_attn_kernel)
  if (!rc) rc = token_qkvg(sn, wqkv, w_g, q_bias, 0.17677669529663687f * kLog2e, buf.q, buf.k, buf.vt, buf.g, M, c_s,
                          NA, stream, "swa_proj_qkvg");
  if (rc) return rc;

  const long long pairs = B * NW * WQ * H;
  {
    KernelTimerScope timed("swa_pair_bias", stream);
    const bf16* zb = static_cast<const bf16*>(z);
    const bf16* wzb = static_cast<const bf16*>(w_z);
    if (c_z == 16)
      launch_swa_bias<16>((int)heads, zb, norm_z_w, norm_z_b, wzb, buf.bias, pairs, (int)H, stream);
    else
      launch_swa_bias<32>((int)heads, zb, norm_z_w, norm_z_b, wzb, buf.bias, pairs, (int)H, stream);
  }
  rc = check_launch("swa_pair_bias");
  if (rc) return rc;
  {
    const size_t key_lds = (size_t)2 * H * sizeof(float);
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(swa_attn_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)key_lds) != hipSuccess)
      return set_error(BIOEMU_ERR_LAUNCH, "swa_attn: cannot set dynamic LDS size");
    KernelTimerScope timed("swa_attn", stream);
    hipLaunchKernelGGL(swa_attn_kernel, dim3((unsigned)NW, (unsigned)((heads + 3) / 4), (unsigned)BM), dim3(256),
                       key_lds, stream, buf.q, buf.k, buf.vt, buf.g, buf.bias, mask, buf.go, (int)NW, (int)H,
                       (int)heads, (int)mult);
  }
  rc = check_launch("swa_attn");
  if (rc) return rc;
  return token_out_proj(buf.go, w_o, s, out, nullptr, M, c_s, c_s, NA, NA, residual != 0, stream, "swa_proj_o");
}
