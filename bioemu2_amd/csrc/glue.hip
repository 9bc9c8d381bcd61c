// Pair-tensor glue on either side of the trunk, for gfx950.
//
// DistogramModule.forward (src/bioemu2/biomoa/modules/embedders.py:191-206):
//   out[b, i, j, :] = (z[b, i, j] + z[b, j, i]) Wd^T + bd
// z + z^T is symmetric, so out[i, j] == out[j, i] exactly: one wave computes
// the pairs (i, j >= i) of a 32-key tile once and writes both orders, so z is
// read once and the output written once.
//
// PairwiseConditioning's input projection (biomoa/modules/diffusion.py:509-525):
//   y = LN_256([z_trunk, rel_pos]) Wp^T  (LayerNorm over the 256 concatenated
//   channels, no Linear bias); the two Transitions that follow run the fused
//   row kernel (transition.hip, hidden = 2 a_z).  The LayerNorm affine is
//   folded into Wp (fold.hip); lanes l and l ^ 32 of a wave hold the z_trunk
//   and rel_pos halves of one pair row.
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int CZ = 128;
constexpr int kThreads = 256;
constexpr int kMaxBins = 128;

// ---------------------------------------------------------------------------
// Distogram.  Wave tile = (b, row i, 32 keys j0 .. j0 + 31); lane (n, hh) holds
// channel chunks 2s + hh of pair (i, j0 + n) (pairtile.h).  Tiles entirely
// below the diagonal exit.  The output is bf16 (OutT = bf16) or fp32 (the
// fp32 accumulator plus the bias, unrounded).
// ---------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(kThreads) void distogram_kernel(const bf16* __restrict__ z, const bf16* __restrict__ wd,
                                                             const float* __restrict__ bd, OutT* __restrict__ out,
                                                             int B, int N, int NB, int NBp) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  stage_weights(wl, wd, NB, NBp);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, hh = lane >> 5;
  const unsigned tiles = (N + 31) / 32;
  const unsigned ntiles = (unsigned)B * N * tiles;
  for (unsigned t = blockIdx.x * 4 + wave; t < ntiles; t += gridDim.x * 4) {
    const TileIdx ti = split_tile(t, tiles, N);
    const int jt = ti.col, i = ti.row, b = ti.b;
    if (jt * 32 + 31 < i) continue;   // wave-uniform: every pair of the tile has j < i
    const int j = jt * 32 + n;
    const bool valid = j < N && j >= i;
    bf16x8 x[8];
    {
      const bf16* zij = z + (((size_t)b * N + i) * N + (valid ? j : i)) * CZ + 8 * hh;
      const bf16* zji = z + (((size_t)b * N + (valid ? j : i)) * N + i) * CZ + 8 * hh;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const bf16x8 a = load8(zij + 16 * s), c = load8(zji + 16 * s);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[s][e] = f2bf(bf2f(a[e]) + bf2f(c[e]));   // one bf16 rounding of z + z^T
      }
    }
    for (int r0 = 0; r0 < NBp; r0 += 32) {
      const f32x16 acc = proj_block_pm(x, wl, r0, n, hh);   // lane (n, hh): bins r0 + 16hh + u of pair (i, j)
      const int c0 = r0 + 16 * hh;
      if (valid && c0 < NB) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = acc[u] + (c0 + u < NB ? bd[c0 + u] : 0.f);
        OutT* o1 = out + (((size_t)b * N + i) * N + j) * NB + c0;
        OutT* o2 = out + (((size_t)b * N + j) * N + i) * NB + c0;
        if constexpr (std::is_same<OutT, float>::value) {
          for (int u = 0; u < 16 && c0 + u < NB; ++u) {
            o1[u] = v[u];
            if (j != i) o2[u] = v[u];
          }
        } else if ((NB & 7) == 0 && c0 + 16 <= NB) {
          store16(o1, v);
          if (j != i) store16(o2, v);
        } else {
          for (int u = 0; u < 16 && c0 + u < NB; ++u) {
            o1[u] = f2bf(v[u]);
            if (j != i) o2[u] = f2bf(v[u]);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pairwise-conditioning input projection: 4 waves x 32 pairs per workgroup;
// folded weights [128][256] (row stride 264) + bias pairs in LDS.  With a
// tail (out_tail != null) the output is written as a residual stream, bf16
// value + int8 tail (common.h), for the transitions that follow.
// ---------------------------------------------------------------------------
constexpr int kCin = 2 * CZ;            // 256 concatenated channels
constexpr int kOut = CZ;                // a_z = 128
constexpr int kLdw2 = kCin + 8;
constexpr int kPcSmem = kOut * kLdw2 * 2 + kOut * 2 * 2;

__global__ __launch_bounds__(kThreads) void pair_cond_proj_kernel(const bf16* __restrict__ zt,
                                                                  const bf16* __restrict__ rel,
                                                                  const bf16* __restrict__ wf,
                                                                  const bf16* __restrict__ cf, bf16* __restrict__ out,
                                                                  int8_t* __restrict__ out_tail, long long P) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  bf16* cl = wl + kOut * kLdw2;
  for (int q = threadIdx.x; q < kOut * (kCin / 8); q += kThreads) {
    const int r = q / (kCin / 8), part = q % (kCin / 8);
    store8(wl + r * kLdw2 + part * 8, load8(wf + (size_t)r * kCin + part * 8));
  }
  for (int q = threadIdx.x; q < 2 * kOut; q += kThreads) cl[q] = cf[q];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 31, hh = lane >> 5;
  const long long p = (long long)blockIdx.x * 128 + wave * 32 + n;
  const bool valid = p < P;
  // lane hh = 0: z_trunk channels 0..127, hh = 1: rel_pos channels (128..255 of the concatenation)
  const bf16* row = (hh == 0 ? zt : rel) + (size_t)(valid ? p : 0) * CZ;
  float v[CZ];
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    bf16x8 raw;
    if (valid) {
      raw = load8(row + 8 * s);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) raw[e] = f2bf(0.f);
    }
    unpack8(raw, v + 8 * s);
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CZ; ++c) sum += v[c];
  sum += __shfl_xor(sum, 32);
  const float mean = sum * (1.0f / kCin);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CZ; ++c) {
    const float d = v[c] - mean;
    ss += d * d;
  }
  ss += __shfl_xor(ss, 32);
  const float rstd = valid ? rsqrtf(ss * (1.0f / kCin) + 1e-5f) : 0.f;
  bf16x8 x[16];
#pragma unroll
  for (int c = 0; c < CZ; ++c) x[c >> 3][c & 7] = f2bf((v[c] - mean) * rstd);
  const bf16x8 xb = bias_step_x(valid, hh);
#pragma unroll
  for (int ob = 0; ob < kOut / 32; ++ob) {
    const int r = ob * 32 + perm32(n);
    const bf16* w = wl + r * kLdw2 + CZ * hh;
    f32x16 acc = zero16();
#pragma unroll
    for (int s = 0; s < 16; ++s) acc = mfma32(load8(w + 8 * s), x[s], acc);
    acc = mfma32(bias_step_w(cl, r, hh), xb, acc);
    // D lane (n, hh): output channel ob*32 + 16hh + u of pair p
    if (valid) {
      float o[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) o[u] = acc[u];
      const size_t off = (size_t)p * kOut + ob * 32 + 16 * hh;
      if (out_tail)
        tail_store16(out + off, out_tail + off, o);
      else
        store16(out + off, o);
    }
  }
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" int bioemu_distogram_fwd(const void* z, const void* w, const float* b, void* out, int64_t B, int64_t N,
                                    int64_t c_z, int64_t num_bins, int out_f32, hipStream_t stream) {
  if (c_z != CZ || num_bins <= 0 || num_bins > kMaxBins)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "distogram: supported c_z = 128, 1 <= num_bins <= %d (got %lld, %lld)",
                     kMaxBins, (long long)c_z, (long long)num_bins);
  if (B <= 0 || N <= 0 || B * N * N > (1LL << 40))
    return set_error(BIOEMU_ERR_INVALID_ARG, "distogram: bad shape B=%lld N=%lld", (long long)B, (long long)N);
  if (!z || !w || !b || !out) return set_error(BIOEMU_ERR_INVALID_ARG, "distogram: null pointer argument");
  if (!aligned16(z) || !aligned16(w) || !aligned16(out))
    return set_error(BIOEMU_ERR_INVALID_ARG, "distogram: tensors must be 16-byte aligned");
  if (out_f32 != 0 && out_f32 != 1)
    return set_error(BIOEMU_ERR_INVALID_ARG, "distogram: out_f32 must be 0 or 1 (got %d)", out_f32);
  const int NBp = (int)round_up(num_bins, 32);
  const size_t smem = (size_t)NBp * kLdw * 2;
  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const long long ntiles = B * N * ((N + 31) / 32);
  if (ntiles >= kMaxTiles) return set_error(BIOEMU_ERR_INVALID_ARG, "distogram: too many pair tiles");
  const unsigned grid = (unsigned)std::max<long long>(1, std::min<long long>(8LL * cus, (ntiles + 3) / 4));
  KernelTimerScope timed("distogram", stream);
  if (out_f32)
    hipLaunchKernelGGL(distogram_kernel<float>, dim3(grid), dim3(kThreads), smem, stream, static_cast<const bf16*>(z),
                       static_cast<const bf16*>(w), b, static_cast<float*>(out), (int)B, (int)N, (int)num_bins, NBp);
  else
    hipLaunchKernelGGL(distogram_kernel<bf16>, dim3(grid), dim3(kThreads), smem, stream, static_cast<const bf16*>(z),
                       static_cast<const bf16*>(w), b, static_cast<bf16*>(out), (int)B, (int)N, (int)num_bins, NBp);
  return check_launch("distogram");
}

extern "C" size_t bioemu_pair_cond_workspace_bytes(int64_t token_z, int64_t c_rel, int64_t a_z) {
  if (token_z != CZ || c_rel != CZ || a_z != kOut) return 0;
  return fold_bytes(kOut, kCin);
}

extern "C" int bioemu_pair_cond_proj_fwd(const void* z_trunk, const void* rel, const float* ln_w, const float* ln_b,
                                         const void* w, void* out, int8_t* out_tail, void* workspace,
                                         size_t workspace_bytes, int64_t P, int64_t token_z, int64_t c_rel,
                                         int64_t a_z, hipStream_t stream) {
  if (token_z != CZ || c_rel != CZ || a_z != kOut)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "pair_cond: supported token_z = rel = a_z = 128 (got %lld, %lld, %lld)",
                     (long long)token_z, (long long)c_rel, (long long)a_z);
  if (P <= 0) return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond: bad row count %lld", (long long)P);
  if (!z_trunk || !rel || !ln_w || !ln_b || !w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond: null pointer argument");
  if (!aligned16(z_trunk) || !aligned16(rel) || !aligned16(w) || !aligned16(out) || !aligned16(workspace) ||
      (out_tail && !aligned16(out_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond: tensors must be 16-byte aligned");
  if (workspace_bytes < bioemu_pair_cond_workspace_bytes(token_z, c_rel, a_z))
    return set_error(BIOEMU_ERR_WORKSPACE, "pair_cond: workspace too small");
  char* base = static_cast<char*>(workspace);
  bf16* wf = reinterpret_cast<bf16*>(base);
  bf16* cf = reinterpret_cast<bf16*>(base + round_up((int64_t)kOut * kCin * 2, 256));
  int rc = launch_fold_ln(w, ln_w, ln_b, wf, cf, kOut, stream, kCin);
  if (rc) return rc;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(pair_cond_proj_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kPcSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "pair_cond: cannot set dynamic LDS size");
  const long long nwg = (P + 127) / 128;
  if (nwg > 0x7fffffffLL) return set_error(BIOEMU_ERR_INVALID_ARG, "pair_cond: too many rows");
  KernelTimerScope timed("pair_cond_proj", stream);
  hipLaunchKernelGGL(pair_cond_proj_kernel, dim3((unsigned)nwg), dim3(kThreads), kPcSmem, stream,
                     static_cast<const bf16*>(z_trunk), static_cast<const bf16*>(rel), wf, cf,
                     static_cast<bf16*>(out), out_tail, (long long)P);
  return check_launch("pair_cond_proj");
}
