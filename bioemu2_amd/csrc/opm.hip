// Fused OuterProductMean for gfx950.
//
// Reference: OuterProductMeanVanilla.forward
// (src/bioemu2/biomoa/ops/outer_product_mean.py:45-75):
//   p = proj_ab(LN(m)); p[~mask] = 0; a, b = chunk(p, 2)            [B,S,N,C_H] each
//   num_valid = mask.any(-1).sum(1).clamp(min=1)   ([B,S,N] mask; 1 for a [B,N] mask)
//   o[b,i,j,c*C_H+d] = sum_s a[b,s,i,c] b[b,s,j,d] / num_valid[b]   (fp32)
//   out = proj_o(o.to(m.dtype)) (+ bias)
// The mean is applied before the cast to the operand dtype, as the reference's
// memory-saving kernel does (src/bioemu2/biomoa/ops/triton/opm.py:114-116).
//
// Kernels:
//   opm_rows  : per batch, the ordered list of MSA rows with any valid entry
//               and its length (= the reference's num_valid before clamping).
//               Rows outside the list are all-zero after the mask, so
//               contracting over the list only is exact.
//   opm_proj  : LN + proj_ab on MFMA; masked entries are zeroed *before* the
//               bias-free projection (0 * W = 0 exactly, the same as
//               masked_fill after it).  Writes aT[b][n][c][r], bT[b][n][d][r]
//               with the compacted row r contiguous (zero for r >= count,
//               rows padded to Sp = S rounded up to 64).
//   opm_fused : one workgroup per (b, 8 i, 8 j) pair tile.  X[(i,c),(j,d)] =
//               sum_r aT[(i,c)][r] bT[(j,d)][r] as one 256 x 256 tile of the
//               NT tile loop (gemm_nt.h: operands copied straight into LDS in
//               64-row stages, double-buffered) over the valid rows rounded
//               up to 64, times 1/num_valid, cast to bf16 into LDS as
//               [pair][c*32+d], then out^T = Wo * X^T + bias (+ z) from LDS on
//               MFMA.
#include <algorithm>

#include "common.h"
#include "gemm_nt.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int CIN = 64;
constexpr int CH = 32;
constexpr int COUT = 128;
constexpr int CH2 = CH * CH;  // 1024

// ---------------------------------------------------------------------------
// Row compaction.  One workgroup per batch.
// ---------------------------------------------------------------------------
constexpr int kRowsThreads = 256;

__global__ __launch_bounds__(kRowsThreads) void opm_rows_kernel(const uint8_t* __restrict__ mask, int* __restrict__ idx,
                                                                int* __restrict__ count, int S, int N) {
  __shared__ int part[kRowsThreads];
  const int b = blockIdx.x;
  const int per = (S + kRowsThreads - 1) / kRowsThreads;
  const int s0 = min(S, (int)threadIdx.x * per), s1 = min(S, s0 + per);
  const uint8_t* mb = mask + (size_t)b * S * N;
  const bool vec = (N % 16 == 0) && ((reinterpret_cast<uintptr_t>(mask) & 15) == 0);
  uint64_t bits = 0;  // per <= 64 rows per thread (S <= 16384)
  int cnt = 0;
  for (int s = s0; s < s1; ++s) {
    const uint8_t* row = mb + (size_t)s * N;
    bool any = false;
    if (vec) {
      for (int t = 0; t < N && !any; t += 16) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + t);
        any = (v.x | v.y | v.z | v.w) != 0;
      }
    } else {
      for (int t = 0; t < N && !any; ++t) any = row[t] != 0;
    }
    if (any) {
      bits |= 1ull << (s - s0);
      ++cnt;
    }
  }
  part[threadIdx.x] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int t = 0; t < kRowsThreads; ++t) {
      const int c = part[t];
      part[t] = run;
      run += c;
    }
    count[b] = run;
  }
  __syncthreads();
  int out = part[threadIdx.x];
  for (int s = s0; s < s1; ++s)
    if (bits >> (s - s0) & 1ull) idx[(size_t)b * S + out++] = s;
}

// ---------------------------------------------------------------------------
// Projection.  Tile = (b, token n, 32 compacted rows).  A 64-channel row is
// held by lanes l and l^32 (channels 32h .. 32h+31, 4 MFMA k-steps).
// ---------------------------------------------------------------------------
constexpr int kProjThreads = 256;

__global__ __launch_bounds__(kProjThreads) void opm_proj_kernel(
    const bf16* __restrict__ m, const uint8_t* __restrict__ mask, const int* __restrict__ idx,
    const int* __restrict__ count, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    const bf16* __restrict__ w_ab, bf16* __restrict__ aT, bf16* __restrict__ bT, int B, int S, int N, int Nt,
    int Sp) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rho = lane & 31, h = lane >> 5;
  const int waves = blockDim.x >> 6;
  const unsigned rtiles = Sp / 32;
  const unsigned ntiles = (unsigned)B * Nt * rtiles;
  for (unsigned t = blockIdx.x * waves + wave; t < ntiles; t += gridDim.x * waves) {
    const TileIdx ti = split_tile(t, rtiles, Nt);
    const int rt = ti.col, n = ti.row, b = ti.b;
    const int r0 = rt * 32;
    const int nv = count[b];
    const int r = r0 + perm32(rho);
    int s = -1;
    if (r < nv && n < N) s = idx[(size_t)b * S + r];
    bool valid = s >= 0;
    if (valid) valid = mask[((size_t)b * S + s) * N + n] != 0;
    float v[32];
    bf16x8 raw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (s >= 0) {
        raw[q] = load8(m + (((size_t)b * S + s) * N + n) * CIN + 32 * h + 8 * q);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) raw[q][e] = f2bf(0.f);
      }
      unpack8(raw[q], v + 8 * q);
    }
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) sum += v[e];
    sum += __shfl_xor(sum, 32);
    const float mean = sum * (1.0f / CIN);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float d = v[e] - mean;
      ss += d * d;
    }
    ss += __shfl_xor(ss, 32);
    const float rstd = rsqrtf(ss * (1.0f / CIN) + 1e-5f);
    bf16x8 xf[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 32 * h + 8 * q + e;
        const float y = (v[8 * q + e] - mean) * rstd * ln_w[c] + ln_b[c];
        xf[q][e] = f2bf(valid ? y : 0.f);  // masked_fill before the bias-free projection
      }
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      f32x16 acc = zero16();
      const bf16* wr = w_ab + (size_t)(which * CH + rho) * CIN + 32 * h;
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = mfma32(xf[q], load8(wr + 8 * q), acc);
      float o[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) o[u] = acc[u];
      bf16* dst = (which ? bT : aT) + (((size_t)b * Nt + n) * CH + rho) * Sp + r0 + 16 * h;
      store16(dst, o);
    }
  }
}

// ---------------------------------------------------------------------------
// proj_o weight in MFMA A-operand fragment order: fragment (eb, ks) of 32
// output rows x 16 inputs is 1 KB contiguous, lane (n, h) holding
// W_o[eb * 32 + perm32(n)][16 ks + 8 h + 0..7], so that each fragment load of
// the fused kernel's epilogue reads whole cache lines.
// ---------------------------------------------------------------------------
constexpr int kWoFrags = (COUT / 32) * (CH2 / 16) * 64;   // 16-byte slots

__global__ __launch_bounds__(256) void opm_wo_tiles_kernel(const bf16* __restrict__ w_o, bf16* __restrict__ wt) {
  const int f = blockIdx.x * 256 + threadIdx.x;
  if (f >= kWoFrags) return;
  const int lane = f & 63, ks = (f >> 6) % (CH2 / 16), eb = f / (64 * (CH2 / 16));
  const int n = lane & 31, h = lane >> 5;
  store8(wt + (size_t)f * 8, load8(w_o + (size_t)(eb * 32 + perm32(n)) * CH2 + 16 * ks + 8 * h));
}

// ---------------------------------------------------------------------------
// Fused contraction + mean + output projection.
// ---------------------------------------------------------------------------
constexpr int kFusedThreads = 512;
constexpr int TI = 8, TJ = 8;            // pair tile
constexpr int LDX = CH2 + 8;             // LDS row stride of the mean tile
constexpr int kFusedSmemB = TI * TJ * LDX * 2;
constexpr int kFusedSmem = kNtSmem > kFusedSmemB ? kNtSmem : kFusedSmemB;

__global__ __launch_bounds__(kFusedThreads) void opm_fused_kernel(
    const bf16* __restrict__ aT, const bf16* __restrict__ bT, const int* __restrict__ count, int mean_rows,
    const bf16* __restrict__ w_t, const float* __restrict__ b_o, const bf16* zres, bf16* out, int8_t* tail, int N, int Nt, int Sp) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* stage = reinterpret_cast<bf16*>(smem);
  bf16* xb = reinterpret_cast<bf16*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * TI, j0 = blockIdx.x * TJ;
  const int nv = count[b];
  const int kend = (nv + kNtBK - 1) / kNtBK * kNtBK;   // rows >= nv of aT / bT are zero

  // X[(i,c),(j,d)] = sum_r aT[(i,c)][r] bT[(j,d)][r]: one 256 x 256 tile of the
  // NT tile loop (gemm_nt.h; operands staged straight into LDS, 64-deep
  // stages), rows Sp apart.  acc[jb][ib], lane (n, h), register u <->
  // row (i,c) = wi*64 + ib*32 + n, column (j,d) = wj*128 + jb*32 + 16h + u.
  f32x16 acc[4][2];
  if (kend > 0) {
    gemm_nt_tile(aT + ((size_t)b * Nt + i0) * CH * Sp, kNtTile, bT + ((size_t)b * Nt + j0) * CH * Sp,
                 bT + ((size_t)b * Nt + j0) * CH * Sp, kNtTile, 0, kend, Sp, stage, acc);
  } else {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) acc[x][y] = zero16();
  }
  __syncthreads();   // the last stage's reads are done before xb overwrites it

  // Mean before the cast: xb[pair (ii, jj)][c*32 + d] = X[(i,c),(j,d)] / num_valid.
  const float inv = mean_rows ? 1.0f / (float)max(nv, 1) : 1.0f;
  const int wi = wave & 3, wj = wave >> 2;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int row = wi * 64 + ib * 32 + n;   // (i, c)
      const int ii = row >> 5, c = row & 31;
      const int jj = wj * 4 + jb;              // column block = one j, d = 16h + u
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = acc[jb][ib][u] * inv;
      store16(xb + (ii * TJ + jj) * LDX + c * CH + 16 * h, v);
    }

  // out^T[e][pair] = Wo[e][:] . xb[pair][:] ; wave -> (e block, pair block).
  // The weight fragments come from L2 (1 KB each, pre-tiled), kPf in flight;
  // the first kPf are requested before the barrier that publishes xb.
  const int eb = wave & 3, pb = wave >> 2;
  const bf16* wfr = w_t + ((size_t)eb * (CH2 / 16) * 64 + lane) * 8;   // fragment ks at wfr + 512 ks
  constexpr int kPf = 32, kSteps = CH2 / 16;
  bf16x8 wq[kPf];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < kPf; ++q) wq[q] = load8(wfr + 512 * q);
  __syncthreads();
  f32x16 y = zero16();
  const bf16* xrow = xb + (pb * 32 + n) * LDX + 8 * h;
#pragma unroll
  for (int ks = 0; ks < kSteps; ++ks) {
    const bf16x8 wc = wq[ks % kPf];
    if (ks + kPf < kSteps) wq[ks % kPf] = load8(wfr + 512 * (ks + kPf));
    y = mfma32(wc, load8(xrow + 16 * ks), y);
    __builtin_amdgcn_sched_barrier(0);   // keeps each load kPf steps ahead of its use
  }
  const int p = pb * 32 + n, ii = p / TJ, jj = p % TJ;
  const int i = i0 + ii, j = j0 + jj;
  if (i >= N || j >= N) return;
  const size_t off = (((size_t)b * N + i) * N + j) * COUT + eb * 32 + 16 * h;
  float v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) v[u] = y[u] + b_o[eb * 32 + 16 * h + u];
  if (zres && tail) {   // residual stream with an int8 tail (common.h), in place
    float zv[16];
    tail_decode16(load8(zres + off), load8(zres + off + 8), load_tail16(tail + off), zv);
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] += zv[u];
    tail_store16(out + off, tail + off, v);
    return;
  }
  if (zres) {
    const bf16x8 r0 = load8(zres + off), r1 = load8(zres + off + 8);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      v[u] += bf2f(r0[u]);
      v[8 + u] += bf2f(r1[u]);
    }
  }
  store16(out + off, v);
}

struct OpmLayout {
  int* idx;
  int* count;
  bf16* aT;
  bf16* bT;
  bf16* wt;   // proj_o weight in fragment order
};

size_t opm_layout(int64_t B, int64_t S, int64_t N, OpmLayout* L, char* base) {
  const size_t Nt = (size_t)round_up(N, 8), Sp = (size_t)round_up(S, 64);
  const size_t idx_b = round_up((size_t)B * S * 4, 256), cnt_b = round_up((size_t)B * 4, 256);
  const size_t ab_b = round_up((size_t)B * Nt * CH * Sp * 2, 256);
  const size_t wt_b = (size_t)kWoFrags * 16;
  if (L) {
    L->idx = reinterpret_cast<int*>(base);
    L->count = reinterpret_cast<int*>(base + idx_b);
    L->aT = reinterpret_cast<bf16*>(base + idx_b + cnt_b);
    L->bT = reinterpret_cast<bf16*>(base + idx_b + cnt_b + ab_b);
    L->wt = reinterpret_cast<bf16*>(base + idx_b + cnt_b + 2 * ab_b);
  }
  return idx_b + cnt_b + 2 * ab_b + wt_b;
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_opm_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_in, int64_t c_hidden) {
  if (B <= 0 || S <= 0 || N <= 0 || c_in != CIN || c_hidden != CH) return 0;
  return opm_layout(B, S, N, nullptr, nullptr);
}

extern "C" int bioemu_opm_fwd(const void* m, const uint8_t* mask, int mean_rows, const float* norm_w,
                              const float* norm_b, const void* w_ab, const void* w_o, const float* b_o,
                              const void* z_res, void* out, int8_t* res_tail, void* workspace,
                              size_t workspace_bytes, int64_t B, int64_t S, int64_t N, int64_t c_in,
                              int64_t c_hidden, int64_t c_out, hipStream_t stream) {
  if (c_in != CIN || c_hidden != CH || c_out != COUT)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "opm: only c_in=64, c_hidden=32, c_out=128 supported (got %lld/%lld/%lld)",
                     (long long)c_in, (long long)c_hidden, (long long)c_out);
  if (B <= 0 || S <= 0 || N <= 0 || S > 16384 || N > 16384 || B > 65535)
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm: bad shape B=%lld S=%lld N=%lld", (long long)B, (long long)S,
                     (long long)N);
  if (!m || !mask || !norm_w || !norm_b || !w_ab || !w_o || !b_o || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm: null pointer argument");
  if (!aligned16(m) || !aligned16(w_ab) || !aligned16(w_o) || !aligned16(out) || !aligned16(workspace) ||
      (z_res && !aligned16(z_res)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm: tensors must be 16-byte aligned");
  if (res_tail && (!z_res || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "opm: res_tail needs z_res and 16-byte alignment");
  if (workspace_bytes < opm_layout(B, S, N, nullptr, nullptr))
    return set_error(BIOEMU_ERR_WORKSPACE, "opm: workspace too small");
  OpmLayout L;
  opm_layout(B, S, N, &L, static_cast<char*>(workspace));
  const int64_t Nt = round_up(N, 8), Sp = round_up(S, 64);
  if (B * Nt * (Sp / 32) >= kMaxTiles) return set_error(BIOEMU_ERR_INVALID_ARG, "opm: too many row tiles");

  {
    KernelTimerScope timed("opm_rows", stream);
    hipLaunchKernelGGL(opm_rows_kernel, dim3((unsigned)B), dim3(kRowsThreads), 0, stream, mask, L.idx, L.count,
                       (int)S, (int)N);
  }
  int rc = check_launch("opm_rows");
  if (rc) return rc;

  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const long long ntiles = B * Nt * (Sp / 32);
  const unsigned grid2 = (unsigned)std::min<long long>(8LL * cus, (ntiles + 3) / 4);
  {
    KernelTimerScope timed("opm_proj", stream);
    hipLaunchKernelGGL(opm_proj_kernel, dim3(grid2), dim3(kProjThreads), 0, stream, static_cast<const bf16*>(m), mask,
                       L.idx, L.count, norm_w, norm_b, static_cast<const bf16*>(w_ab), L.aT, L.bT, (int)B, (int)S,
                       (int)N, (int)Nt, (int)Sp);
  }
  rc = check_launch("opm_proj");
  if (rc) return rc;

  {
    KernelTimerScope timed("opm_wo_tiles", stream);
    hipLaunchKernelGGL(opm_wo_tiles_kernel, dim3((kWoFrags + 255) / 256), dim3(256), 0, stream,
                       static_cast<const bf16*>(w_o), L.wt);
  }
  rc = check_launch("opm_wo_tiles");
  if (rc) return rc;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(opm_fused_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kFusedSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "opm_fused: cannot set dynamic LDS size");
  dim3 g3((unsigned)(Nt / TJ), (unsigned)(Nt / TI), (unsigned)B);
  {
    KernelTimerScope timed("opm_fused", stream);
    hipLaunchKernelGGL(opm_fused_kernel, g3, dim3(kFusedThreads), kFusedSmem, stream, L.aT, L.bT, L.count, mean_rows,
                       L.wt, b_o, static_cast<const bf16*>(z_res), static_cast<bf16*>(out),
                       res_tail, (int)N, (int)Nt, (int)Sp);
  }
  return check_launch("opm_fused");
}
