// Batched bf16 NT GEMM on MFMA: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k].
//
// Used for the per-channel triangle contraction, where both operands are
// channel-major [z = b*D + d][row][k] planes with k contiguous.  M = N = K = n,
// n a multiple of 256, so the kernel has no edge handling; callers zero-pad.
//
// Tiling: 256 x 256 workgroup tile, BK = 32, 512 threads = 8 waves in a
// 4 (i) x 2 (j) grid, each wave 64 (i) x 128 (j) = 2 x 4 MFMA 32x32x16 blocks.
// Per 16-deep k-step a wave reads 6 operand fragments for 8 MFMAs.  The MFMA
// A operand is the B tile (rows j, permuted with perm32) and the B operand is
// the A tile (rows i), so an accumulator lane holds 16 consecutive j of one i:
// C rows are written as 32-byte runs straight from registers.
// Global -> LDS staging is double-buffered through registers (the next k-tile
// is fetched while the current one is multiplied).  The k reduction order is
// fixed (k = 0, 1, ... in 16-wide MFMA steps), so appending zero-valued k
// columns never changes a result bit.
//
// Workgroup -> (plane, tile) mapping is XCD-aware: consecutive workgroup ids
// are dispatched round-robin over the 8 XCDs, so ids are regrouped such that
// all tiles of one plane land on one XCD and share its L2.
#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int LDK = BK + 8;          // LDS row stride (bf16): 80 B, conflict-free 16-B reads
constexpr int kThreads = 512;
constexpr int kStage = (BM + BN) * LDK;
constexpr int kSmem = 2 * kStage * 2;
constexpr int kXcds = 8;

__global__ __launch_bounds__(kThreads) void bgemm_nt_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                            bf16* __restrict__ C, int n, int batch) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);

  // XCD-aware mapping: workgroup w runs on XCD w % 8; give each XCD a
  // contiguous range of (plane, tile) work items.
  const int tiles = (n / BM) * (n / BN);
  const int total = tiles * batch;
  const int w = blockIdx.x;
  const int per_xcd = (total + kXcds - 1) / kXcds;
  const int item = (w % kXcds) * per_xcd + w / kXcds;
  if (item >= total) return;
  const int z = item / tiles, t = item % tiles;
  const int ti = t / (n / BN), tj = t % (n / BN);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;

  const size_t plane = (size_t)n * n;
  const bf16* Ab = A + (size_t)z * plane + (size_t)ti * BM * n;
  const bf16* Bb = B + (size_t)z * plane + (size_t)tj * BN * n;

  // Staging: each operand tile is 256 rows x 4 chunks of 16 B = 1024 chunks;
  // thread tid moves chunks tid and tid + 512 of each.
  bf16x8 ra[2], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int q = it * kThreads + tid;
      const int row = q >> 2, part = q & 3;
      ra[it] = load8(Ab + (size_t)row * n + k0 + part * 8);
      rb[it] = load8(Bb + (size_t)row * n + k0 + part * 8);
    }
  };
  auto lstore = [&](int st) {
    bf16* sa = smem + st * kStage;
    bf16* sb = sa + BM * LDK;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int q = it * kThreads + tid;
      const int row = q >> 2, part = q & 3;
      store8(sa + row * LDK + part * 8, ra[it]);
      store8(sb + row * LDK + part * 8, rb[it]);
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = zero16();

  const int nk = n / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  const int jrow = perm32(ln);
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) gload((kt + 1) * BK);
    const bf16* sa = smem + cur * kStage;
    const bf16* sb = sa + BM * LDK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8 fj[4], fi[2];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) fj[jb] = load8(sb + (wj * 128 + jb * 32 + jrow) * LDK + ks * 16 + 8 * lh);
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) fi[ib] = load8(sa + (wi * 64 + ib * 32 + ln) * LDK + ks * 16 + 8 * lh);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = mfma32(fj[jb], fi[ib], acc[jb][ib]);
    }
    if (more) lstore(cur ^ 1);
    __syncthreads();
  }

  // D lane (ln, lh) of block (jb, ib): i = wi*64 + ib*32 + ln, j = wj*128 + jb*32 + 16lh + u.
  bf16* Cb = C + (size_t)z * plane + (size_t)(ti * BM) * n + tj * BN;
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) {
    bf16* crow = Cb + (size_t)(wi * 64 + ib * 32 + ln) * n + wj * 128 + 16 * lh;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = acc[jb][ib][u];
      store16(crow + jb * 32, v);
    }
  }
}

}  // namespace

int launch_bgemm_nt(const void* A, const void* B, void* C, int64_t batch, int64_t n, hipStream_t stream) {
  if (n % kGemmTile != 0 || n <= 0 || batch <= 0 || batch * (n / BM) * (n / BN) > (1ll << 31) - 1) {
    return set_error(BIOEMU_ERR_INVALID_ARG, "bgemm_nt: bad shape batch=%lld n=%lld", (long long)batch,
                     (long long)n);
  }
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(bgemm_nt_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          kSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "bgemm_nt: cannot set dynamic LDS size");
  const long long total = batch * (n / BM) * (n / BN);
  const long long grid = (total + kXcds - 1) / kXcds * kXcds;
  KernelTimerScope timed("bgemm_nt", stream);
  hipLaunchKernelGGL(bgemm_nt_kernel, dim3((unsigned)grid), dim3(kThreads), kSmem, stream,
                     static_cast<const bf16*>(A), static_cast<const bf16*>(B), static_cast<bf16*>(C), (int)n,
                     (int)batch);
  return check_launch("bgemm_nt");
}

}  // namespace bioemu
