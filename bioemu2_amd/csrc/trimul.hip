// Triangle multiplicative update (outgoing / incoming) for gfx950.
//
// Reference: TriangleMultiplicationFull.forward
// (src/bioemu2/biomoa/ops/triangle_multiplication.py:89-99).
//
// Pipeline (all bf16 in HBM, fp32 math in registers):
//   1. trimul_proj_in : LN_in -> [p_in | g_in] (128 -> 2x256) -> a,b = p*sigmoid(g)
//                       -> mask select -> channel-major planes a[d][i][k], b[d][j][k]
//                       (the incoming direction writes the transposed frame).
//   2. bgemm_nt       : o[d][i][j] = sum_k a[d][i][k] * b[d][j][k]   (MFMA, fp32 acc)
//   3. trimul_out     : LN_out(o) -> p_out, LN_in(x) -> g_out, out = p*sigmoid(g) (+x)
// Padded planes (Np = N rounded up to 128) are zero in every padded row and
// column, so the contraction needs no edge handling and padding never changes
// a valid output bit.
#include "common.h"
#include "internal.h"

namespace bioemu {
namespace {

constexpr int D = 128;           // pair channels (c_z)
constexpr int LDX = D + 8;       // LDS row stride (bf16) of a pair tile
constexpr int kThreads = 256;    // 4 waves
constexpr int kTilePairs = 256;  // pairs per workgroup: 4 frame rows x 64 frame columns

// ---------------------------------------------------------------------------
// Stage 1: LN_in + gated input projection + mask, channel-major output.
// Frame tile: rows i0..i0+3 (one per wave) x columns k0..k0+63.
// Outgoing reads x[i][k]; incoming reads x[k][i] (frame = transpose).
// ---------------------------------------------------------------------------
template <bool kOutgoing>
__global__ __launch_bounds__(kThreads) void trimul_proj_in_kernel(
    const bf16* __restrict__ x, const uint8_t* __restrict__ mask, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ p_w, const bf16* __restrict__ g_w,
    bf16* __restrict__ ab, int B, int N, int Np) {
  __shared__ __attribute__((aligned(16))) bf16 xt[kTilePairs * LDX];
  __shared__ uint8_t mk[kTilePairs];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, lh = lane >> 5;
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * 4;
  const int k0 = blockIdx.x * 64;
  const size_t pair_base = (size_t)b * N * N;

  // Coalesced tile load: 16 threads per pair (16 B each).  Outgoing walks the
  // 64 frame columns of one x row (16 KB contiguous); incoming walks the 4
  // frame rows, which are 4 consecutive pairs of one x row (1 KB contiguous).
#pragma unroll 4
  for (int it = 0; it < 16; ++it) {
    const int q = it * kThreads + tid;
    const int part = q & 15;
    int w, kk;
    if (kOutgoing) {
      kk = (q >> 4) & 63;
      w = q >> 10;
    } else {
      w = (q >> 4) & 3;
      kk = q >> 6;
    }
    const int i = i0 + w, k = k0 + kk;
    bf16x8 v;
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = f2bf(0.f);
    if (i < N && k < N) {
      const int r = kOutgoing ? i : k, c = kOutgoing ? k : i;
      v = load8(x + (pair_base + (size_t)r * N + c) * D + part * 8);
    }
    store8(xt + (w * 64 + kk) * LDX + part * 8, v);
  }
  {
    const int w = tid >> 6, kk = tid & 63;
    const int i = i0 + w, k = k0 + kk;
    uint8_t valid = 0;
    if (i < N && k < N) {
      const int r = kOutgoing ? i : k, c = kOutgoing ? k : i;
      valid = mask[pair_base + (size_t)r * N + c] != 0;
    }
    mk[tid] = valid;
  }
  __syncthreads();
  layernorm_row_lds<D>(xt + tid * LDX, ln_w, ln_b, 1e-5f);
  __syncthreads();

  // MFMA: rows = this wave's 64 pairs (2 blocks of 32), cols = 32 channels.
  bf16x8 afr[2][D / 16];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      afr[rb][s] = load8(xt + (wave * 64 + rb * 32 + ln) * LDX + s * 16 + lh * 8);

  const size_t plane = (size_t)Np * Np;
  for (int which = 0; which < 2; ++which) {
    for (int cc = 0; cc < D / 32; ++cc) {
      const int wrow = which * D + cc * 32 + ln;
      bf16x8 bp[D / 16], bg[D / 16];
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        bp[s] = load8(p_w + (size_t)wrow * D + s * 16 + lh * 8);
        bg[s] = load8(g_w + (size_t)wrow * D + s * 16 + lh * 8);
      }
      const int ch = cc * 32 + ln;
      bf16* dst_plane = ab + ((size_t)(which * B + b) * D + ch) * plane + (size_t)(i0 + wave) * Np + k0;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        f32x16 accp = zero16(), accg = zero16();
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          accp = mfma32(afr[rb][s], bp[s], accp);
          accg = mfma32(afr[rb][s], bg[s], accg);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float o[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int kk = rb * 32 + 8 * r + 4 * lh + c;
            const float v = accp[4 * r + c] * sigmoidf_fast(accg[4 * r + c]);
            o[c] = mk[wave * 64 + kk] ? v : 0.f;  // masked_fill semantics (select, not multiply)
          }
          *reinterpret_cast<bf16x4*>(dst_plane + rb * 32 + 8 * r + 4 * lh) = pack4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Stage 3: LN_out(o) -> p_out, LN_in(x) -> g_out, out = p * sigmoid(g) (+ x).
// Output tile: rows i0..i0+3 (one per wave) x columns j0..j0+63, channel-last.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void trimul_out_kernel(
    const bf16* __restrict__ o, const bf16* x, const float* __restrict__ ln_in_w,
    const float* __restrict__ ln_in_b, const float* __restrict__ ln_out_w,
    const float* __restrict__ ln_out_b, const bf16* __restrict__ p_w, const bf16* __restrict__ g_w,
    bf16* out, int N, int Np, int residual) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* ot = reinterpret_cast<bf16*>(smem);  // [256][LDX] contraction result, pair-major
  bf16* xt = ot + kTilePairs * LDX;          // [256][LDX] x tile

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, lh = lane >> 5;
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * 4;
  const int j0 = blockIdx.x * 64;
  const size_t plane = (size_t)Np * Np;
  const size_t pair_base = (size_t)b * N * N;

  // o planes are channel-major: read 128-byte row pieces, transpose into LDS.
#pragma unroll 4
  for (int it = 0; it < 16; ++it) {
    const int q = it * kThreads + tid;
    const int part = q & 7, w = (q >> 3) & 3, d = q >> 5;
    const bf16x8 v = load8(o + ((size_t)b * D + d) * plane + (size_t)(i0 + w) * Np + j0 + part * 8);
#pragma unroll
    for (int t = 0; t < 8; ++t) ot[(w * 64 + part * 8 + t) * LDX + d] = v[t];
  }
#pragma unroll 4
  for (int it = 0; it < 16; ++it) {
    const int q = it * kThreads + tid;
    const int part = q & 15, jj = (q >> 4) & 63, w = q >> 10;
    const int i = i0 + w, j = j0 + jj;
    bf16x8 v;
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = f2bf(0.f);
    if (i < N && j < N) v = load8(x + (pair_base + (size_t)i * N + j) * D + part * 8);
    store8(xt + (w * 64 + jj) * LDX + part * 8, v);
  }
  __syncthreads();
  layernorm_row_lds<D>(ot + tid * LDX, ln_out_w, ln_out_b, 1e-5f);
  layernorm_row_lds<D>(xt + tid * LDX, ln_in_w, ln_in_b, 1e-5f);
  __syncthreads();

  const int i = i0 + wave;
  for (int cc = 0; cc < D / 32; ++cc) {
    bf16x8 ap[D / 16], ag[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      ap[s] = load8(p_w + (size_t)(cc * 32 + ln) * D + s * 16 + lh * 8);
      ag[s] = load8(g_w + (size_t)(cc * 32 + ln) * D + s * 16 + lh * 8);
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int prow = wave * 64 + cb * 32 + ln;
      f32x16 accp = zero16(), accg = zero16();
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        accp = mfma32(ap[s], load8(ot + prow * LDX + s * 16 + lh * 8), accp);
        accg = mfma32(ag[s], load8(xt + prow * LDX + s * 16 + lh * 8), accg);
      }
      const int j = j0 + cb * 32 + ln;
      if (i < N && j < N) {
        bf16* dst = out + (pair_base + (size_t)i * N + j) * D + cc * 32;
        const bf16* res = x + (pair_base + (size_t)i * N + j) * D + cc * 32;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] = accp[4 * r + c] * sigmoidf_fast(accg[4 * r + c]);
          const int ch = 8 * r + 4 * lh;
          if (residual) {
            const bf16x4 xr = *reinterpret_cast<const bf16x4*>(res + ch);
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] += bf2f(xr[c]);
          }
          *reinterpret_cast<bf16x4*>(dst + ch) = pack4(v[0], v[1], v[2], v[3]);
        }
      }
    }
  }
}

constexpr int kOutSmem = 2 * kTilePairs * LDX * 2;

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_trimul_workspace_bytes(int64_t B, int64_t N, int64_t Dc) {
  if (B <= 0 || N <= 0 || Dc <= 0) return 0;
  const int64_t Np = round_up(N, kGemmTile);
  return (size_t)(3 * B * Dc * Np * Np) * sizeof(bf16);
}

extern "C" int bioemu_trimul_fwd(const void* x, const uint8_t* mask, const float* norm_in_w,
                                 const float* norm_in_b, const void* p_in_w, const void* g_in_w,
                                 const float* norm_out_w, const float* norm_out_b,
                                 const void* p_out_w, const void* g_out_w, void* out,
                                 void* workspace, size_t workspace_bytes, int64_t B, int64_t N,
                                 int64_t Dc, int outgoing, int residual, hipStream_t stream) {
  if (Dc != D) return set_error(BIOEMU_ERR_UNSUPPORTED, "trimul: channel dim %lld unsupported (must be 128)", (long long)Dc);
  if (B <= 0 || N <= 0 || B > 65535 || N > 16384)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: bad shape B=%lld N=%lld", (long long)B, (long long)N);
  if (!x || !mask || !norm_in_w || !norm_in_b || !p_in_w || !g_in_w || !norm_out_w || !norm_out_b ||
      !p_out_w || !g_out_w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(p_in_w) || !aligned16(g_in_w) ||
      !aligned16(p_out_w) || !aligned16(g_out_w) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: x/out/weights/workspace must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: out may alias x only with residual=1");
  const size_t need = bioemu_trimul_workspace_bytes(B, N, Dc);
  if (workspace_bytes < need)
    return set_error(BIOEMU_ERR_WORKSPACE, "trimul: workspace %zu < required %zu", workspace_bytes, need);

  const int64_t Np = round_up(N, kGemmTile);
  const size_t plane_elems = (size_t)(B * D * Np * Np);
  bf16* ab = static_cast<bf16*>(workspace);
  bf16* ob = ab + 2 * plane_elems;

  dim3 g1((unsigned)(Np / 64), (unsigned)(Np / 4), (unsigned)B);
  {
  KernelTimerScope timed("trimul_proj_in", stream);
  if (outgoing) {
    hipLaunchKernelGGL(trimul_proj_in_kernel<true>, g1, dim3(kThreads), 0, stream,
                       static_cast<const bf16*>(x), mask, norm_in_w, norm_in_b,
                       static_cast<const bf16*>(p_in_w), static_cast<const bf16*>(g_in_w), ab, (int)B,
                       (int)N, (int)Np);
  } else {
    hipLaunchKernelGGL(trimul_proj_in_kernel<false>, g1, dim3(kThreads), 0, stream,
                       static_cast<const bf16*>(x), mask, norm_in_w, norm_in_b,
                       static_cast<const bf16*>(p_in_w), static_cast<const bf16*>(g_in_w), ab, (int)B,
                       (int)N, (int)Np);
  }
  }
  int rc = check_launch("trimul_proj_in");
  if (rc) return rc;
  rc = launch_bgemm_nt(ab, ab + plane_elems, ob, B * D, Np, stream);
  if (rc) return rc;

  if (hipFuncSetAttribute(reinterpret_cast<const void*>(trimul_out_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kOutSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "trimul_out: cannot set dynamic LDS size");
  dim3 g3((unsigned)((N + 63) / 64), (unsigned)((N + 3) / 4), (unsigned)B);
  KernelTimerScope timed("trimul_out", stream);
  hipLaunchKernelGGL(trimul_out_kernel, g3, dim3(kThreads), kOutSmem, stream, ob,
                     static_cast<const bf16*>(x), norm_in_w, norm_in_b, norm_out_w, norm_out_b,
                     static_cast<const bf16*>(p_out_w), static_cast<const bf16*>(g_out_w),
                     static_cast<bf16*>(out), (int)N, (int)Np, residual);
  return check_launch("trimul_out");
}
