// Batched bf16 NT GEMM on MFMA: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k].
//
// Used for the per-channel triangle contraction, where both operands are
// channel-major [z = b*D + d][row][k] planes with k contiguous.  M = N = K = n,
// n a multiple of 256, so the kernel has no edge handling; callers zero-pad.
// The tile main loop (256 x 256, BK = 64, LDS staged by direct copies) is
// gemm_nt_tile (gemm_nt.h); this file adds the plain row-major store.
// Workgroup -> (plane, tile) mapping is XCD-aware: all tiles of one plane land
// on one XCD and share its L2.
#include "common.h"
#include "gemm_nt.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

__global__ __launch_bounds__(kNtThreads) void bgemm_nt_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                              bf16* __restrict__ C, int n, int batch) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  const int tiles = (n / kNtTile) * (n / kNtTile);
  const int item = nt_item(tiles * batch);
  if (item < 0) return;
  const int z = item / tiles, t = item % tiles;
  const int ti = t / (n / kNtTile), tj = t % (n / kNtTile);
  const size_t plane = (size_t)n * n;

  f32x16 acc[4][2];
  gemm_nt_tile(A + z * plane + (size_t)ti * kNtTile * n, B + z * plane + (size_t)tj * kNtTile * n, n, smem, acc);

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;
  bf16* Cb = C + z * plane + (size_t)(ti * kNtTile) * n + tj * kNtTile;
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
  if (n % kGemmTile != 0 || n <= 0 || batch <= 0 || batch * (n / kNtTile) * (n / kNtTile) > (1ll << 31) - 1 ||
      (long long)kNtTile * n * 2 > 0xffffffffLL) {
    return set_error(BIOEMU_ERR_INVALID_ARG, "bgemm_nt: bad shape batch=%lld n=%lld", (long long)batch,
                     (long long)n);
  }
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(bgemm_nt_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          kNtSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "bgemm_nt: cannot set dynamic LDS size");
  const long long total = batch * (n / kNtTile) * (n / kNtTile);
  const long long grid = (total + kNtXcds - 1) / kNtXcds * kNtXcds;
  KernelTimerScope timed("bgemm_nt", stream);
  hipLaunchKernelGGL(bgemm_nt_kernel, dim3((unsigned)grid), dim3(kNtThreads), kNtSmem, stream,
                     static_cast<const bf16*>(A), static_cast<const bf16*>(B), static_cast<bf16*>(C), (int)n,
                     (int)batch);
  return check_launch("bgemm_nt");
}

}  // namespace bioemu
