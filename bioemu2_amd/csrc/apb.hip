// Attention with pair bias over the single representation, for gfx950.
//
// Reference: AttentionPairBias.forward
// (src/bioemu2/biomoa/ops/attention_pair_bias.py:128-225), non-fused bias
// branch (_proj_z_fused, :114-117):
//   s' = LN_s(s) if initial_norm;  q,k,v = chunk(s' Wqkv^T);  q += q_bias
//   g = sigmoid(s' Wg^T);  bias[b,h,i,j] = (LN_z(z) Wz^T)[b,i,j,h]
//   A = q k^T / sqrt(d) + bias (broadcast over the multiplicity M);
//   A[..., ~mask_j] = -1e6 (replace);  o = softmax_j(A) v
//   out = (g * o) Wo^T            (+ s when residual != 0)
//
// Kernels: token LN / GEMMs for the per-token projections (token.hip); the
// pair-bias pre-pass below reads z exactly once at full-chip parallelism
// and writes a bf16 [B][H][Np][Np] bias (1/8 of z's bytes at c_z = 128,
// H = 16); the flash kernel runs one wave per (batch*M, head, 32 queries)
// with an online softmax over 32-key blocks and writes g * o.
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int CZ = 128;
constexpr int kBiasThreads = 256;

// bias[b][h][i][j] = LN(z[b][i][j]) . Wz[h] for i, j < Np (zero pair rows outside [0, N)),
// with the LayerNorm folded into Wz (wf, cf from launch_fold_ln).
__global__ __launch_bounds__(kBiasThreads) void pair_bias_kernel(const bf16* __restrict__ z,
                                                                 const bf16* __restrict__ wf,
                                                                 const bf16* __restrict__ cf, bf16* __restrict__ bias,
                                                                 int B, int N, int Np, int H) {
  __shared__ __attribute__((aligned(16))) bf16 wl[32 * kLdw];
  __shared__ bf16 cl[64];
  stage_weights(wl, wf, H, 32);
  stage_bias(cl, cf, H, 32);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rho = lane & 31, h = lane >> 5;
  const int waves = blockDim.x >> 6;
  const unsigned tiles_per_row = Np / 32;
  const unsigned ntiles = (unsigned)B * Np * tiles_per_row;
  const size_t plane = (size_t)Np * Np;
  // Software pipeline over this wave's tiles: iteration t issues tile
  // t + stride's z loads, projects tile t, normalises tile t + stride and only
  // then stores tile t's bias, so the wait for the loads (vector-memory
  // counters retire in issue order) covers only stores issued a whole tile
  // earlier.  The loads are unconditional (pair 0 for slots outside the
  // sequence, zeroed when normalised).
  const unsigned stride = gridDim.x * waves;
  bf16x8 raw[8];
  auto fetch = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tiles_per_row, Np);
    const int kk = ti.col * 32 + perm32(rho);
    const bool valid = ti.row < N && kk < N;
    const bf16* row = z + (((size_t)ti.b * N + (valid ? ti.row : 0)) * N + (valid ? kk : 0)) * CZ + 8 * h;
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) raw[s8] = load8(row + 16 * s8);
  };
  bf16x8 x[8], xb;
  auto prepare = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tiles_per_row, Np);
    const int kk = ti.col * 32 + perm32(rho);
    const bool valid = ti.row < N && kk < N;
    float v[64];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) unpack8(valid ? raw[s8] : bf16x8{}, v + 8 * s8);
    normalize_half_row(v, valid, x);
    xb = bias_step_x(valid, h);
  };

  unsigned t = blockIdx.x * waves + wave;
  if (t < ntiles) {
    fetch(t);
    prepare(t);
  }
  for (; t < ntiles; t += stride) {
    const unsigned tn = t + stride;
    if (tn < ntiles) fetch(tn);
    const TileIdx ti = split_tile(t, tiles_per_row, Np);
    const f32x16 acc = proj_block_cm_f(x, xb, wl, cl, 0, rho, h);
    bf16x8 o[2];   // tile t's bias, packed while tile t + stride is normalised
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      o[0][u] = f2bf(acc[u]);
      o[1][u] = f2bf(acc[8 + u]);
    }
    if (tn < ntiles) prepare(tn);
    if (rho < H) {
      bf16* dst = bias + ((size_t)ti.b * H + rho) * plane + (size_t)ti.row * Np + ti.col * 32 + 16 * h;
      store8(dst, o[0]);
      store8(dst + 8, o[1]);
    }
  }
}

// ---------------------------------------------------------------------------
// Flash kernel.  Block = (32 queries, 4 heads, batch*M row bm); wave w owns
// head 4*blockIdx.y + w.  Head dim 24 is zero-padded to 32 for the 16-deep
// MFMA k-steps (k-step 1, half 1 carries d = 24..31 = 0).
// Same register dataflow as the triangle-attention flash kernel:
// S^T = K Q^T (lane (n, hh) holds keys k0 + 16hh + u of query q0 + n),
// O^T = V^T P^T (lane holds d = 16hh + u).
// ---------------------------------------------------------------------------
constexpr int DH = 24;
constexpr int kMaxMaskN = 16384;

__global__ __launch_bounds__(256) void apb_flash_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                        const bf16* __restrict__ vt, const bf16* __restrict__ g,
                                                        const bf16* __restrict__ bias,
                                                        const uint8_t* __restrict__ mask, bf16* __restrict__ go,
                                                        int N, int Np, int H, int mult) {
  __shared__ __attribute__((aligned(16))) uint8_t mrow[kMaxMaskN];
  const int bm = blockIdx.z, b = bm / mult;
  const int CS = H * DH;
  for (int t = threadIdx.x; t < Np; t += blockDim.x) mrow[t] = (t < N) ? (mask[(size_t)b * N + t] != 0) : 0;
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, hh = lane >> 5;
  const int hd = blockIdx.y * 4 + wave;
  if (hd >= H) return;  // after the only barrier
  const int q0 = blockIdx.x * 32;
  const float qk_scale = kLog2e / sqrtf((float)DH);
  const float masked_logit = -1e6f * kLog2e;

  bf16x8 zero8;
#pragma unroll
  for (int t = 0; t < 8; ++t) zero8[t] = f2bf(0.f);

  const bf16* qrow = q + ((size_t)bm * Np + q0 + n) * CS + hd * DH;
  const bf16x8 qf0 = load8(qrow + 8 * hh);
  const bf16x8 qf1 = hh == 0 ? load8(qrow + 16) : zero8;

  f32x16 o = zero16();
  float m = -INFINITY, l = 0.f;
  const bf16* kbase = k + (size_t)bm * Np * CS + hd * DH;
  const int dslot = perm32(n);
  const bf16* vbase = vt + ((size_t)bm * CS + hd * DH + (dslot < DH ? dslot : 0)) * Np;
  const bf16* brow = bias + (((size_t)b * H + hd) * Np + q0 + n) * Np;

  for (int k0 = 0; k0 < Np; k0 += 32) {
    const bf16* kr = kbase + (size_t)(k0 + perm32(n)) * CS;
    f32x16 s = zero16();
    s = mfma32(load8(kr + 8 * hh), qf0, s);
    s = mfma32(hh == 0 ? load8(kr + 16) : zero8, qf1, s);
    const bf16x8 b0 = load8(brow + k0 + 16 * hh), b1 = load8(brow + k0 + 16 * hh + 8);
    const uint4 mk = *reinterpret_cast<const uint4*>(mrow + k0 + 16 * hh);
    const uint32_t mw[4] = {mk.x, mk.y, mk.z, mk.w};
    float t[16];
    float bmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float bv = bf2f(u < 8 ? b0[u] : b1[u - 8]);
      float x = s[u] * qk_scale + bv * kLog2e;
      if (((mw[u >> 2] >> (8 * (u & 3))) & 0xff) == 0) x = masked_logit;
      if (k0 + 16 * hh + u >= N) x = -INFINITY;
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
    const bf16* vp = vbase + k0 + 16 * hh;
    const bool dvalid = dslot < DH;
    o = mfma32(dvalid ? load8(vp) : zero8, pb[0], o);
    o = mfma32(dvalid ? load8(vp + 8) : zero8, pb[1], o);
  }

  const float inv = 1.0f / (l + __shfl_xor(l, 32));
  const size_t off = ((size_t)bm * Np + q0 + n) * CS + hd * DH + 16 * hh;
  if (hh == 0) {
    const bf16x8 g0 = load8(g + off), g1 = load8(g + off + 8);
    float v[16];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      v[u] = bf2f(g0[u]) * (o[u] * inv);
      v[8 + u] = bf2f(g1[u]) * (o[8 + u] * inv);
    }
    store16(go + off, v);
  } else {
    const bf16x8 g0 = load8(g + off);
    bf16x8 r;
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = f2bf(bf2f(g0[u]) * (o[u] * inv));
    store8(go + off, r);
  }
}

struct ApbBuffers {
  bf16 *sn, *q, *k, *vt, *g, *go, *bias, *wf, *cf;
};

size_t apb_layout(int64_t B, int64_t BM, int64_t N, int64_t CS, int64_t H, ApbBuffers* buf, char* base) {
  const size_t Np = (size_t)round_up(N, 32);
  const size_t tok = round_up(BM * Np * CS * 2, 256);
  const size_t bias_bytes = round_up((size_t)B * H * Np * Np * 2, 256);
  if (buf) {
    char* p = base;
    buf->sn = reinterpret_cast<bf16*>(p);
    p += tok;
    buf->q = reinterpret_cast<bf16*>(p);
    p += tok;
    buf->k = reinterpret_cast<bf16*>(p);
    p += tok;
    buf->vt = reinterpret_cast<bf16*>(p);
    p += tok;
    buf->g = reinterpret_cast<bf16*>(p);
    p += tok;
    buf->go = reinterpret_cast<bf16*>(p);
    p += tok;
    buf->bias = reinterpret_cast<bf16*>(p);
    p += bias_bytes;
    buf->wf = reinterpret_cast<bf16*>(p);
    buf->cf = reinterpret_cast<bf16*>(p + round_up((size_t)32 * 128 * 2, 256));
  }
  return 6 * tok + bias_bytes + fold_bytes(32);
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_apb_workspace_bytes(int64_t B, int64_t mult, int64_t N, int64_t c_s, int64_t H) {
  if (B <= 0 || mult <= 0 || N <= 0 || c_s <= 0 || H <= 0) return 0;
  return apb_layout(B, B * mult, N, c_s, H, nullptr, nullptr);
}

extern "C" int bioemu_apb_fwd(const void* s, const void* z, const uint8_t* mask, const float* norm_s_w,
                              const float* norm_s_b, const void* w_qkv, const float* q_bias, const void* w_g,
                              const float* norm_z_w, const float* norm_z_b, const void* w_z, const void* w_o,
                              void* out, int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t B,
                              int64_t mult, int64_t N, int64_t c_s, int64_t c_z, int64_t H, int residual,
                              hipStream_t stream) {
  if (c_z != CZ || H <= 0 || H > 32 || c_s != H * DH || (c_s != 384 && c_s != 128))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "apb: supported shapes are c_z=128 and head dim 24 with c_s in {128, 384} (got c_s=%lld c_z=%lld H=%lld)",
                     (long long)c_s, (long long)c_z, (long long)H);
  if (B <= 0 || mult <= 0 || N <= 0 || N > kMaxMaskN || B * mult > 65535)
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb: bad shape B=%lld M=%lld N=%lld", (long long)B, (long long)mult,
                     (long long)N);
  if (!s || !z || !mask || !w_qkv || !q_bias || !w_g || !norm_z_w || !w_z || !w_o || !out || !workspace ||
      (norm_s_w == nullptr) != (norm_s_b == nullptr))
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb: null pointer argument");
  if (!aligned16(s) || !aligned16(z) || !aligned16(out) || !aligned16(w_qkv) || !aligned16(w_g) ||
      !aligned16(w_z) || !aligned16(w_o) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb: tensors must be 16-byte aligned");
  if (out == s && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb: out may alias s only with residual=1");
  if (res_tail && (!residual || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "apb: res_tail needs residual=1 and 16-byte alignment");
  const int64_t BM = B * mult;
  if (workspace_bytes < apb_layout(B, BM, N, c_s, H, nullptr, nullptr))
    return set_error(BIOEMU_ERR_WORKSPACE, "apb: workspace too small");
  ApbBuffers buf;
  apb_layout(B, BM, N, c_s, H, &buf, static_cast<char*>(workspace));
  const int64_t Np = round_up(N, 32);
  const int64_t M = BM * Np;
  const bf16* wqkv = static_cast<const bf16*>(w_qkv);

  int rc = token_layernorm(s, norm_s_w, norm_s_b, buf.sn, BM, N, Np, c_s, stream);
  if (!rc) rc = token_gemm(kEpiStoreId, false, buf.sn, wqkv, nullptr, q_bias, nullptr, buf.q, M, c_s, c_s, N, Np, Np,
                           stream, "apb_proj_q");
  if (!rc) rc = token_gemm(kEpiStoreId, false, buf.sn, wqkv + c_s * c_s, nullptr, nullptr, nullptr, buf.k, M, c_s,
                           c_s, N, Np, Np, stream, "apb_proj_k");
  if (!rc) rc = token_gemm(kEpiStoreId, true, buf.sn, wqkv + 2 * c_s * c_s, nullptr, nullptr, nullptr, buf.vt, M,
                           c_s, c_s, N, Np, Np, stream, "apb_proj_v");
  if (!rc) rc = token_gemm(kEpiSigmoidId, false, buf.sn, w_g, nullptr, nullptr, nullptr, buf.g, M, c_s, c_s, N, Np,
                           Np, stream, "apb_proj_g");
  if (rc) return rc;

  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const long long ntiles = B * Np * (Np / 32);
  if (ntiles >= kMaxTiles) return set_error(BIOEMU_ERR_INVALID_ARG, "apb: too many pair tiles");
  const unsigned grid1 = (unsigned)std::min<long long>(4LL * cus, (ntiles + 3) / 4);
  rc = launch_fold_ln(w_z, norm_z_w, norm_z_b, buf.wf, buf.cf, H, stream);
  if (rc) return rc;
  {
    KernelTimerScope timed("apb_pair_bias", stream);
    hipLaunchKernelGGL(pair_bias_kernel, dim3(grid1), dim3(kBiasThreads), 0, stream, static_cast<const bf16*>(z),
                       buf.wf, buf.cf, buf.bias, (int)B, (int)N, (int)Np, (int)H);
  }
  rc = check_launch("apb_pair_bias");
  if (rc) return rc;
  {
    KernelTimerScope timed("apb_flash", stream);
    hipLaunchKernelGGL(apb_flash_kernel, dim3((unsigned)(Np / 32), (unsigned)((H + 3) / 4), (unsigned)BM), dim3(256),
                       0, stream, buf.q, buf.k, buf.vt, buf.g, buf.bias, mask, buf.go, (int)N, (int)Np, (int)H,
                       (int)mult);
  }
  rc = check_launch("apb_flash");
  if (rc) return rc;
  return token_gemm(residual ? kEpiResidualId : kEpiStoreId, false, buf.go, w_o, nullptr, nullptr, s, out, M, c_s,
                    c_s, N, Np, N, stream, "apb_proj_o", res_tail);
}
