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

// bias[b][h][i][j] = log2(e) * LN(z[b][i][j]) . Wz[h] for i, j < Np (zero pair rows outside
// [0, N)), with the LayerNorm folded into Wz (wf, cf from launch_fold_ln).  The
// attention's softmax runs in base 2, so the bias is stored in log2 units.
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
      o[0][u] = f2bf(acc[u] * kLog2e);
      o[1][u] = f2bf(acc[8 + u] * kLog2e);
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
// Flash kernel.  Workgroup = (128 queries, one head, batch*M row bm): wave w
// owns queries q0 = 128 blockIdx.x + 32 w of head blockIdx.y.  Per 32-key
// block the workgroup stages K [32 keys][d] and V^T [d][32 keys] once in LDS
// (double-buffered, head dim 24 zero-padded to 32 there), so its four waves
// share them; each wave fetches its own bias rows one block ahead.
// Same register dataflow as the triangle-attention flash kernel:
// S^T = K Q^T (lane (n, hh) holds keys k0 + 16hh + u of query q0 + n),
// O^T = V^T P^T (lane holds d = 16hh + u).
// ---------------------------------------------------------------------------
constexpr int DH = 24;
constexpr float kQScale = 0.20412414523193154f * kLog2e;   // log2(e) / sqrt(DH)
constexpr int kMaxMaskN = 16384;
constexpr int kFlashQ = 128;                  // queries per workgroup
constexpr int kKvLd = 40;                     // LDS row stride (bf16) of the K and V^T tiles
constexpr int kKvTile = 32 * kKvLd;           // one tile: 32 rows
constexpr int kKvStage = 2 * kKvTile;         // K then V^T
constexpr int kKvChunks = 32 * 3 + 24 * 4;    // 16-byte global chunks per block: K 32 x 3, V^T 24 x 4

__global__ __launch_bounds__(256) void apb_flash_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                        const bf16* __restrict__ vt, const bf16* __restrict__ g,
                                                        const bf16* __restrict__ bias,
                                                        const uint8_t* __restrict__ mask, bf16* __restrict__ go,
                                                        int N, int Np, int H, int mult) {
  // Per key t: the logit is x = kv[t] * (q.k + bias) + c0[t], i.e. unchanged
  // for a valid key (kv = 1, c0 = 0), replaced by the reference's -1e6 (in
  // log2 units) for a masked one (kv = 0), and -inf past N (no such key).
  // (dynamic LDS: kv[Np] then c0[Np])
  extern __shared__ __attribute__((aligned(16))) float key_terms[];
  __shared__ __attribute__((aligned(16))) bf16 kvs[2 * kKvStage];
  float* kvl = key_terms;
  float* c0l = key_terms + Np;
  const int bm = blockIdx.z, b = bm / mult, hd = blockIdx.y;
  const int CS = H * DH;
  const int tid = threadIdx.x;
  const float masked_logit = -1e6f * kLog2e;
  for (int t = tid; t < Np; t += blockDim.x) {
    const bool valid = t < N && mask[(size_t)b * N + t] != 0;
    kvl[t] = valid ? 1.f : 0.f;
    c0l[t] = valid ? 0.f : t < N ? masked_logit : -INFINITY;
  }
  // zero the padding of both stages once (d 24..31 of K rows, V^T rows 24..31);
  // the staging below never writes it
  for (int e = tid; e < 2 * kKvStage; e += blockDim.x) {
    const int w = e % kKvStage, row = (w % kKvTile) / kKvLd, col = w % kKvLd;
    const bool is_k = w < kKvTile;
    if ((is_k && col >= DH) || (!is_k && row >= DH)) kvs[e] = f2bf(0.f);
  }

  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int q0 = blockIdx.x * kFlashQ + 32 * wave;
  const bool active = q0 < Np;   // idle waves stage tiles and meet every barrier
  const int qr = active ? q0 + n : n;

  bf16x8 zero8;
#pragma unroll
  for (int t = 0; t < 8; ++t) zero8[t] = f2bf(0.f);
  const bf16* qrow = q + ((size_t)bm * Np + qr) * CS + hd * DH;
  const bf16x8 qf0 = load8(qrow + 8 * hh);
  const bf16x8 qf1 = hh == 0 ? load8(qrow + 16) : zero8;

  // Staging: thread tid < 96 moves K chunk (key tid / 3, d 8 (tid % 3)),
  // 96 <= tid < 192 V^T chunk (d (tid - 96) / 4, keys 8 ((tid - 96) % 4)).
  const bool stager = tid < kKvChunks;
  const bool kpart = tid < 96;
  const int srow = kpart ? tid / 3 : (tid - 96) / 4, spart = kpart ? tid % 3 : (tid - 96) % 4;
  const bf16* ksrc = k + ((size_t)bm * Np + srow) * CS + hd * DH + 8 * spart;
  const bf16* vsrc = vt + ((size_t)bm * CS + hd * DH + srow) * Np + 8 * spart;
  const int sdst = (kpart ? 0 : kKvTile) + srow * kKvLd + 8 * spart;
  bf16x8 sreg = zero8;
  auto gload = [&](int kb) {
    if (stager) sreg = kpart ? load8(ksrc + (size_t)kb * CS) : load8(vsrc + kb);
  };
  auto lstore = [&](int st) {
    if (stager) store8(kvs + st * kKvStage + sdst, sreg);
  };
  const bf16* brow = bias + (((size_t)b * H + hd) * Np + qr) * Np + 16 * hh;
  bf16x8 bc0 = load8(brow), bc1 = load8(brow + 8);   // bias of the block being consumed

  gload(0);
  lstore(0);
  __syncthreads();

  f32x16 o = zero16();
  float m = -INFINITY, l = 0.f;
  const int kslot = perm32(n);   // K row / V^T row (d) of this lane's MFMA operand
  int st = 0;
  for (int k0 = 0; k0 < Np; k0 += 32) {
    const int kn = k0 + 32 < Np ? k0 + 32 : k0;   // the last block refetches itself
    gload(kn);
    const bf16x8 bn0 = load8(brow + kn), bn1 = load8(brow + kn + 8);
    const bf16* ks = kvs + st * kKvStage;
    const bf16* vs = ks + kKvTile;
    f32x16 s = zero16();
    s = mfma32(load8(ks + kslot * kKvLd + 8 * hh), qf0, s);
    s = mfma32(load8(ks + kslot * kKvLd + 16 + 8 * hh), qf1, s);
    const float4* kv4 = reinterpret_cast<const float4*>(kvl + k0 + 16 * hh);
    const float4* c04 = reinterpret_cast<const float4*>(c0l + k0 + 16 * hh);
    float kv[16], c0[16];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 a = kv4[e], c = c04[e];
      kv[4 * e] = a.x, kv[4 * e + 1] = a.y, kv[4 * e + 2] = a.z, kv[4 * e + 3] = a.w;
      c0[4 * e] = c.x, c0[4 * e + 1] = c.y, c0[4 * e + 2] = c.z, c0[4 * e + 3] = c.w;
    }
    float t[16];
    float bmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      // q carries log2(e)/sqrt(d) and the bias log2(e): s + bias is the logit in log2 units
      const float x = __builtin_fmaf(s[u] + bf2f(u < 8 ? bc0[u] : bc1[u - 8]), kv[u], c0[u]);
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
    o = mfma32(load8(vs + kslot * kKvLd + 16 * hh), pb[0], o);
    o = mfma32(load8(vs + kslot * kKvLd + 16 * hh + 8), pb[1], o);
    bc0 = bn0;
    bc1 = bn1;
    lstore(st ^ 1);
    st ^= 1;
    __syncthreads();
  }
  if (!active) return;

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
  if (rc) return rc;
  // q carries the attention's softmax scale in base 2 (apb_flash_kernel)
  rc = token_qkvg(buf.sn, wqkv, w_g, q_bias, kQScale, buf.q, buf.k, buf.vt, buf.g, M, c_s, Np, stream,
                  "apb_proj_qkvg");
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
    const size_t key_lds = (size_t)2 * Np * sizeof(float);   // <= 128 KB (N <= 16384)
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(apb_flash_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)key_lds) != hipSuccess)
      return set_error(BIOEMU_ERR_LAUNCH, "apb_flash: cannot set dynamic LDS size");
    KernelTimerScope timed("apb_flash", stream);
    hipLaunchKernelGGL(apb_flash_kernel, dim3((unsigned)((Np + kFlashQ - 1) / kFlashQ), (unsigned)H, (unsigned)BM), dim3(256),
                       key_lds, stream, buf.q, buf.k, buf.vt, buf.g, buf.bias, mask, buf.go, (int)N, (int)Np, (int)H,
                       (int)mult);
  }
  rc = check_launch("apb_flash");
  if (rc) return rc;
  return token_out_proj(buf.go, w_o, s, out, res_tail, M, c_s, c_s, Np, N, residual != 0, stream, "apb_proj_o");
}
