// The PairMixer trunk's glue around its layers, for gfx950.
//
// Recycling (src/bioemu2/biomoa/modules/pairmixer.py:275-296): before every
// trunk pass
//   s = s_init + s_recycle(s_norm(s))      token rows, 384 -> 384
//   z = z_init + z_recycle(z_norm(z))      pair rows,  128 -> 128
// with LayerNorm (affine, eps 1e-5) and bias-free Linear layers (:186-191).
// Both are "out = base + W LN(x)" over rows; the pair form is one HBM-bound
// pass (x, base in, out written) with the LayerNorm folded into the weights
// and the 128x128 product on MFMA; the token form is the token LayerNorm and
// the token GEMM with its residual epilogue (token.hip).
//
// Unconditional branch (classifier-free guidance, pairmixer.py:266-273):
//   z = z_init + uncond_transition(z_norm(z_init))
// is the token LayerNorm kernel over the pair rows (z_norm, affine, written
// bf16 into the workspace) and the fused row transition with z_init (and its
// tail) as the residual base.
//
// MSA input embedding (PairMixerMSAModule.forward, pairmixer.py:591-599):
//   m[b,r,t,:] = msa_proj(cat(msa, has_deletion, deletion_value[, msa_paired]))
//              + s_proj(emb)[b,t,:]
// with bias-free Linear layers (:527-532).  s_proj(emb) is computed once per
// token (fp32), then every MSA row adds its feature projection; m is written
// as a bf16 value with an int8 tail (common.h), the MSA stream's form.
#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int C = kPairC;   // 128 pair channels
constexpr int kThreads = 256;
constexpr int kSmem = C * kLdw * 2 + C * 2 * 2;

// ---------------------------------------------------------------------------
// out[p] = base[p] + W LN(x[p]) over tiles of 32 pair rows per wave.  The
// folded weights W' = W diag(gamma) and the bias W beta (hi, lo) sit in LDS;
// a lane (n, h) loads channel chunks 2s + h of pair p0 + n (pairtile.h), and
// the pair-major product leaves it 16 consecutive output channels of that pair, so base,
// its tail and the output are 32-byte contiguous per lane.  out may alias x
// or base: a pair's row is read entirely before the lane that owns it writes.
// ---------------------------------------------------------------------------
template <bool kBaseTail, bool kOutTail>
__global__ __launch_bounds__(kThreads) void pair_ln_linear_kernel(const bf16* x, const bf16* __restrict__ wf,
                                                                  const bf16* __restrict__ cf, const bf16* base,
                                                                  const int8_t* base_tail, bf16* out,
                                                                  int8_t* out_tail, long long P) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  bf16* cl = wl + C * kLdw;
  stage_weights(wl, wf, C, C);
  stage_bias(cl, cf, C, C);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const long long tiles = (P + 31) / 32;
  const long long stride = (long long)gridDim.x * (kThreads / 64);
  for (long long t = (long long)blockIdx.x * (kThreads / 64) + wave; t < tiles; t += stride) {
    const long long p = t * 32 + n;
    const bool valid = p < P;
    const size_t row = (size_t)(valid ? p : 0) * C;
    float v[64];
    load_half_row_f32(x + row, h, valid, v);
    bf16x8 xn[8];
    normalize_half_row(v, valid, xn);
    const bf16x8 xb = bias_step_x(valid, h);
#pragma unroll
    for (int ob = 0; ob < C / 32; ++ob) {
      const f32x16 acc = proj_block_pm_f(xn, xb, wl, cl, ob * 32, n, h);
      const size_t off = row + ob * 32 + 16 * h;
      float o[16], b[16];
      if (kBaseTail) {
        tail_decode16(load8(base + off), load8(base + off + 8), load_tail16(base_tail + off), b);
      } else {
        unpack8(load8(base + off), b);
        unpack8(load8(base + off + 8), b + 8);
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) o[u] = acc[u] + b[u];
      if (valid) {
        if (kOutTail)
          tail_store16(out + off, out_tail + off, o);
        else
          store16(out + off, o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MSA embedding.  sproj: one thread per (token, output channel), fp32 dot over
// the E input features.  msa_embed: one thread per MSA position (b, r, t):
// the F = F0 + 2 (+1) features are read once, the [C][F] weight sits in LDS,
// and the 64 outputs plus the token's s_proj row are written as value + tail
// (kF32: as fp32 values, for a run with autocast off).
// ---------------------------------------------------------------------------
constexpr int kMsaC = 64;
constexpr int kMaxFeat = 64;

__global__ __launch_bounds__(kThreads) void msa_sproj_kernel(const float* __restrict__ emb,
                                                             const float* __restrict__ ws, float* __restrict__ sp,
                                                             long long BT, int E) {
  const long long idx = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= BT * kMsaC) return;
  const long long bt = idx / kMsaC;
  const int c = (int)(idx % kMsaC);
  const float* e = emb + bt * E;
  const float* w = ws + (size_t)c * E;
  float acc = 0.f;
  for (int k = 0; k < E; ++k) acc = __builtin_fmaf(w[k], e[k], acc);
  sp[idx] = acc;
}

template <bool kF32>
__global__ __launch_bounds__(kThreads) void msa_embed_kernel(const float* __restrict__ msa,
                                                             const float* __restrict__ has_del,
                                                             const float* __restrict__ del_val,
                                                             const float* __restrict__ paired,
                                                             const float* __restrict__ wm, const float* __restrict__ sp,
                                                             void* __restrict__ m_out, int8_t* __restrict__ m_tail,
                                                             long long positions, int R, int T, int F0) {
  __shared__ float wl[kMsaC * kMaxFeat];
  const int F = F0 + 2 + (paired ? 1 : 0);
  for (int q = threadIdx.x; q < kMsaC * F; q += kThreads) wl[q] = wm[q];
  __syncthreads();
  const long long pos = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (pos >= positions) return;
  const long long b = pos / ((long long)R * T);
  const int t = (int)(pos % T);
  // 64 fp32 accumulators seeded with the token's s_proj row; features
  // streamed once, k outermost (the weight reads are LDS broadcasts).
  float o[kMsaC];
  const float* spr = sp + ((size_t)b * T + t) * kMsaC;
#pragma unroll
  for (int c = 0; c < kMsaC; ++c) o[c] = spr[c];
  const float* src = msa + pos * F0;
#pragma unroll 1
  for (int k = 0; k < F; ++k) {
    const float fk = k < F0 ? src[k] : k == F0 ? has_del[pos] : k == F0 + 1 ? del_val[pos] : paired[pos];
#pragma unroll
    for (int c = 0; c < kMsaC; ++c) o[c] = __builtin_fmaf(wl[c * F + k], fk, o[c]);
  }
  if (kF32) {
    float* m = static_cast<float*>(m_out) + pos * kMsaC;
#pragma unroll
    for (int c0 = 0; c0 < kMsaC; c0 += 4) *reinterpret_cast<f32x4*>(m + c0) = f32x4{o[c0], o[c0 + 1], o[c0 + 2], o[c0 + 3]};
    return;
  }
  bf16* m = static_cast<bf16*>(m_out);
#pragma unroll
  for (int c0 = 0; c0 < kMsaC; c0 += 16) tail_store16(m + pos * kMsaC + c0, m_tail + pos * kMsaC + c0, o + c0);
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_pair_ln_linear_workspace_bytes(int64_t Dc) { return Dc == C ? fold_bytes(C) : 0; }

extern "C" int bioemu_pair_ln_linear_fwd(const void* x, const float* norm_w, const float* norm_b, const void* w,
                                         const void* base, const int8_t* base_tail, void* out, int8_t* out_tail,
                                         void* workspace, size_t workspace_bytes, int64_t P, int64_t Dc,
                                         hipStream_t stream) {
  if (Dc != C) return set_error(BIOEMU_ERR_UNSUPPORTED, "pair_ln_linear: only 128 channels (got %lld)", (long long)Dc);
  if (P <= 0 || P >= kMaxTiles * 32) return set_error(BIOEMU_ERR_INVALID_ARG, "pair_ln_linear: bad row count %lld",
                                                      (long long)P);
  if (!x || !norm_w || !w || !base || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pair_ln_linear: null pointer argument");
  if (!aligned16(x) || !aligned16(w) || !aligned16(base) || !aligned16(out) || !aligned16(workspace) ||
      (base_tail && !aligned16(base_tail)) || (out_tail && !aligned16(out_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "pair_ln_linear: buffers must be 16-byte aligned");
  if (workspace_bytes < fold_bytes(C)) return set_error(BIOEMU_ERR_WORKSPACE, "pair_ln_linear: workspace too small");
  bf16* wf = static_cast<bf16*>(workspace);
  bf16* cf = reinterpret_cast<bf16*>(static_cast<char*>(workspace) + round_up((int64_t)C * C * 2, 256));
  int rc = launch_fold_ln(w, norm_w, norm_b, wf, cf, C, stream);
  if (rc) return rc;
  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const long long tiles = (P + 31) / 32;
  const long long grid = std::min<long long>((long long)cus * 4, (tiles + 3) / 4);
  auto* k = base_tail ? (out_tail ? pair_ln_linear_kernel<true, true> : pair_ln_linear_kernel<true, false>)
                      : (out_tail ? pair_ln_linear_kernel<false, true> : pair_ln_linear_kernel<false, false>);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, kSmem) !=
      hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "pair_ln_linear: cannot set dynamic LDS size");
  {
    KernelTimerScope timed("pair_ln_linear", stream);
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kThreads), kSmem, stream, static_cast<const bf16*>(x), wf, cf,
                       static_cast<const bf16*>(base), base_tail, static_cast<bf16*>(out), out_tail, (long long)P);
  }
  return check_launch("pair_ln_linear");
}

extern "C" size_t bioemu_token_ln_linear_workspace_bytes(int64_t M, int64_t Dc) {
  if (M <= 0 || Dc <= 0) return 0;
  return (size_t)round_up(round_up(M, 32) * Dc * 2, 256);
}

extern "C" int bioemu_token_ln_linear_fwd(const void* x, const float* norm_w, const float* norm_b, const void* w,
                                          const void* base, const int8_t* base_tail, void* out, int8_t* out_tail,
                                          void* workspace, size_t workspace_bytes, int64_t M, int64_t Dc,
                                          hipStream_t stream) {
  if (M <= 0 || Dc <= 0 || Dc % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "token_ln_linear: width %lld unsupported (a multiple of 32)",
                     (long long)Dc);
  if (!x || !norm_w || !w || !base || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "token_ln_linear: null pointer argument");
  if ((base_tail != nullptr) != (out_tail != nullptr))
    return set_error(BIOEMU_ERR_INVALID_ARG, "token_ln_linear: base_tail and out_tail go together");
  if (!aligned16(x) || !aligned16(w) || !aligned16(base) || !aligned16(out) || !aligned16(workspace) ||
      (out_tail && (!aligned16(out_tail) || !aligned16(base_tail))))
    return set_error(BIOEMU_ERR_INVALID_ARG, "token_ln_linear: buffers must be 16-byte aligned");
  if (workspace_bytes < bioemu_token_ln_linear_workspace_bytes(M, Dc))
    return set_error(BIOEMU_ERR_WORKSPACE, "token_ln_linear: workspace too small");
  const int64_t Mp = round_up(M, 32);
  bf16* xn = static_cast<bf16*>(workspace);
  int rc = token_layernorm(x, norm_w, norm_b, xn, 1, M, Mp, Dc, stream);
  if (rc) return rc;
  // The residual epilogue reads and rewrites one tail buffer: give it base's tail first.
  if (out_tail && out_tail != base_tail &&
      hipMemcpyAsync(out_tail, base_tail, (size_t)M * Dc, hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "token_ln_linear: tail copy failed");
  return token_gemm(kEpiResidualId, false, xn, w, nullptr, nullptr, base, out, Mp, Dc, Dc, M, Mp, M, stream,
                    "token_ln_linear", out_tail);
}

extern "C" size_t bioemu_trunk_uncond_workspace_bytes(int64_t P, int64_t Dc, int64_t hidden) {
  const size_t fold = bioemu_transition_pair_workspace_bytes(Dc, hidden);
  if (P <= 0 || Dc != C || fold == 0) return 0;
  return (size_t)round_up(P * Dc * 2, 256) + fold;
}

extern "C" int bioemu_trunk_uncond_fwd(const void* z_init, const int8_t* z_init_tail, const float* z_norm_w,
                                       const float* z_norm_b, const float* t_norm_w, const float* t_norm_b,
                                       const void* fc1_w, const void* fc2_w, const void* fc3_w, void* out,
                                       int8_t* out_tail, void* workspace, size_t workspace_bytes, int64_t P,
                                       int64_t Dc, int64_t hidden, hipStream_t stream) {
  if (Dc != C || (hidden != 4 * Dc && hidden != 2 * Dc))
    return set_error(BIOEMU_ERR_UNSUPPORTED, "trunk_uncond: only 128 channels with hidden 512 or 256 (got %lld, %lld)",
                     (long long)Dc, (long long)hidden);
  if (P <= 0 || P > 0x7fffffffLL)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond: bad row count %lld", (long long)P);
  if (!z_init || !z_norm_w || !z_norm_b || !t_norm_w || !t_norm_b || !fc1_w || !fc2_w || !fc3_w || !out ||
      !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond: null pointer argument");
  if ((z_init_tail != nullptr) != (out_tail != nullptr))
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond: z_init_tail and out_tail go together");
  if (!aligned16(z_init) || !aligned16(out) || !aligned16(workspace) ||
      (out_tail && (!aligned16(out_tail) || !aligned16(z_init_tail))))
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond: buffers must be 16-byte aligned");
  if (out == z_init && out_tail != z_init_tail)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trunk_uncond: in place, out_tail must be z_init_tail");
  const size_t need = bioemu_trunk_uncond_workspace_bytes(P, Dc, hidden);
  if (workspace_bytes < need)
    return set_error(BIOEMU_ERR_WORKSPACE, "trunk_uncond: workspace %zu < required %zu", workspace_bytes, need);
  char* p = static_cast<char*>(workspace);
  void* zn = p;
  const size_t zn_bytes = (size_t)round_up(P * Dc * 2, 256);
  int rc = token_layernorm(z_init, z_norm_w, z_norm_b, zn, 1, P, P, Dc, stream);
  if (rc) return rc;
  // The residual epilogue reads and rewrites one tail buffer: give it z_init's tail first.
  if (out_tail && out_tail != z_init_tail &&
      hipMemcpyAsync(out_tail, z_init_tail, (size_t)P * Dc, hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "trunk_uncond: tail copy failed");
  return transition_pair_res(zn, z_init, t_norm_w, t_norm_b, fc1_w, fc2_w, fc3_w, out, out_tail, p + zn_bytes,
                             workspace_bytes - zn_bytes, P, Dc, hidden, 1, 1, stream);
}

extern "C" size_t bioemu_msa_embed_workspace_bytes(int64_t B, int64_t T) {
  if (B <= 0 || T <= 0) return 0;
  return (size_t)round_up(B * T * kMsaC * 4, 256);
}

static int msa_embed(const float* msa, const float* has_deletion, const float* deletion_value,
                     const float* msa_paired, const float* emb, const float* w_msa, const float* w_s, void* m,
                     int8_t* m_tail, bool f32, void* workspace, size_t workspace_bytes, int64_t B, int64_t R,
                     int64_t T, int64_t F0, int64_t E, int64_t msa_s, hipStream_t stream) {
  if (msa_s != kMsaC)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "msa_embed: only msa_s = 64 (got %lld)", (long long)msa_s);
  if (B <= 0 || R <= 0 || T <= 0 || F0 <= 0 || E <= 0 || F0 + 3 > kMaxFeat)
    return set_error(BIOEMU_ERR_INVALID_ARG, "msa_embed: bad shape B=%lld R=%lld T=%lld F0=%lld E=%lld",
                     (long long)B, (long long)R, (long long)T, (long long)F0, (long long)E);
  if (!msa || !has_deletion || !deletion_value || !emb || !w_msa || !w_s || !m || (!f32 && !m_tail) || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "msa_embed: null pointer argument");
  if (!aligned16(m) || (!f32 && !aligned16(m_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "msa_embed: m and its tail must be 16-byte aligned");
  if (workspace_bytes < bioemu_msa_embed_workspace_bytes(B, T))
    return set_error(BIOEMU_ERR_WORKSPACE, "msa_embed: workspace too small");
  float* sp = static_cast<float*>(workspace);
  const long long bt = B * T;
  {
    KernelTimerScope timed("msa_sproj", stream);
    hipLaunchKernelGGL(msa_sproj_kernel, dim3((unsigned)((bt * kMsaC + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       stream, emb, w_s, sp, bt, (int)E);
  }
  int rc = check_launch("msa_sproj");
  if (rc) return rc;
  const long long positions = B * R * T;
  {
    KernelTimerScope timed("msa_embed", stream);
    const dim3 grid((unsigned)((positions + kThreads - 1) / kThreads));
    if (f32)
      hipLaunchKernelGGL(msa_embed_kernel<true>, grid, dim3(kThreads), 0, stream, msa, has_deletion, deletion_value,
                         msa_paired, w_msa, sp, m, nullptr, positions, (int)R, (int)T, (int)F0);
    else
      hipLaunchKernelGGL(msa_embed_kernel<false>, grid, dim3(kThreads), 0, stream, msa, has_deletion, deletion_value,
                         msa_paired, w_msa, sp, m, m_tail, positions, (int)R, (int)T, (int)F0);
  }
  return check_launch("msa_embed");
}

extern "C" int bioemu_msa_embed_fwd(const float* msa, const float* has_deletion, const float* deletion_value,
                                    const float* msa_paired, const float* emb, const float* w_msa, const float* w_s,
                                    void* m, int8_t* m_tail, void* workspace, size_t workspace_bytes, int64_t B,
                                    int64_t R, int64_t T, int64_t F0, int64_t E, int64_t msa_s, hipStream_t stream) {
  return msa_embed(msa, has_deletion, deletion_value, msa_paired, emb, w_msa, w_s, m, m_tail, false, workspace,
                   workspace_bytes, B, R, T, F0, E, msa_s, stream);
}

extern "C" int bioemu_msa_embed_fwd_f32(const float* msa, const float* has_deletion, const float* deletion_value,
                                        const float* msa_paired, const float* emb, const float* w_msa,
                                        const float* w_s, float* m, void* workspace, size_t workspace_bytes,
                                        int64_t B, int64_t R, int64_t T, int64_t F0, int64_t E, int64_t msa_s,
                                        hipStream_t stream) {
  return msa_embed(msa, has_deletion, deletion_value, msa_paired, emb, w_msa, w_s, m, nullptr, true, workspace,
                   workspace_bytes, B, R, T, F0, E, msa_s, stream);
}
