// Batched bf16 NT GEMM on MFMA: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k].
//
// Used for the per-channel triangle contraction, where both operands are
// channel-major [z = b*D + d][row][k] planes with k contiguous.  M = N = K = n,
// n a multiple of 128, so the kernel has no edge handling; callers zero-pad.
//
// Tiling: 128x128 block tile, BK = 64, 256 threads = 4 waves in a 2x2 grid,
// each wave owns a 64x64 sub-tile = 2x2 MFMA 32x32x16 blocks.  Global->LDS
// staging is double-buffered with a register prefetch of the next k-tile.
// The k reduction order is fixed (k = 0, 1, ... in 16-wide MFMA steps), so
// appending zero-valued k columns never changes a result bit.
#include "common.h"
#include "internal.h"

namespace bioemu {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;    // LDS row stride (bf16) of the operand tiles
constexpr int LDC = BN + 8;    // LDS row stride (bf16) of the output staging tile
constexpr int kThreads = 256;
constexpr int kOperandBytes = 2 * (BM + BN) * LDK * 2;
constexpr int kOutBytes = BM * LDC * 2;
constexpr int kSmemBytes = kOperandBytes > kOutBytes ? kOperandBytes : kOutBytes;

__global__ __launch_bounds__(kThreads) void bgemm_nt_kernel(const bf16* __restrict__ A,
                                                            const bf16* __restrict__ B,
                                                            bf16* __restrict__ C, int n) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  bf16* As = reinterpret_cast<bf16*>(smem);            // [2][BM][LDK]
  bf16* Bs = As + 2 * BM * LDK;                        // [2][BN][LDK]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ln = lane & 31, lh = lane >> 5;

  const size_t plane = (size_t)n * n;
  const bf16* Ab = A + (size_t)blockIdx.z * plane + (size_t)blockIdx.y * BM * n;
  const bf16* Bb = B + (size_t)blockIdx.z * plane + (size_t)blockIdx.x * BN * n;

  // Each thread moves 4 16-byte chunks of A and 4 of B per k-tile.
  bf16x8 ra[4], rb[4];
  auto gload = [&](int kt) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int q = it * kThreads + tid;
      const int row = q >> 3, part = q & 7;
      ra[it] = load8(Ab + (size_t)row * n + kt * BK + part * 8);
      rb[it] = load8(Bb + (size_t)row * n + kt * BK + part * 8);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int q = it * kThreads + tid;
      const int row = q >> 3, part = q & 7;
      store8(As + (buf * BM + row) * LDK + part * 8, ra[it]);
      store8(Bs + (buf * BN + row) * LDK + part * 8, rb[it]);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();

  const int nk = n / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const bf16* Ac = As + cur * BM * LDK;
    const bf16* Bc = Bs + cur * BN * LDK;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        af[mi] = load8(Ac + (wm * 64 + mi * 32 + ln) * LDK + s * 16 + lh * 8);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        bfr[ni] = load8(Bc + (wn * 64 + ni * 32 + ln) * LDK + s * 16 + lh * 8);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // Stage the bf16 tile through LDS for 16-byte coalesced row stores.
  bf16* Cs = reinterpret_cast<bf16*>(smem);  // [BM][LDC]
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int row = wm * 64 + mi * 32 + 8 * r + 4 * lh + c;
          const int col = wn * 64 + ni * 32 + ln;
          Cs[row * LDC + col] = f2bf(acc[mi][ni][4 * r + c]);
        }
  __syncthreads();
  bf16* Cb = C + (size_t)blockIdx.z * plane + (size_t)blockIdx.y * BM * n + (size_t)blockIdx.x * BN;
#pragma unroll
  for (int it = 0; it < (BM * BN / 8) / kThreads; ++it) {
    const int q = it * kThreads + tid;
    const int row = q >> 4, part = q & 15;
    store8(Cb + (size_t)row * n + part * 8, load8(Cs + row * LDC + part * 8));
  }
}

}  // namespace

int launch_bgemm_nt(const void* A, const void* B, void* C, int64_t batch, int64_t n,
                    hipStream_t stream) {
  if (n % kGemmTile != 0 || n <= 0 || batch <= 0 || batch > 65535) {
    return set_error(BIOEMU_ERR_INVALID_ARG, "bgemm_nt: bad shape batch=%lld n=%lld",
                     (long long)batch, (long long)n);
  }
  dim3 grid((unsigned)(n / BN), (unsigned)(n / BM), (unsigned)batch);
  KernelTimerScope timed("bgemm_nt", stream);
  hipLaunchKernelGGL(bgemm_nt_kernel, grid, dim3(kThreads), 0, stream,
                     static_cast<const bf16*>(A), static_cast<const bf16*>(B), static_cast<bf16*>(C),
                     (int)n);
  return check_launch("bgemm_nt");
}

}  // namespace bioemu
