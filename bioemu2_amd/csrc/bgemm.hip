// Batched bf16 NT GEMM on MFMA: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k].
//
// Used for the per-channel triangle contraction, where both operands are
// channel-major [z = b*D + d][row][k] planes with k contiguous.  M = N = K = n,
// n a multiple of 256, so the kernel has no edge handling; callers zero-pad.
// Tiles are 256 x 256 with BK = 64, staged into LDS by direct copies and
// multiplied by the k-tile body of gemm_nt.h.
//
// Persistent: one workgroup per CU walks a list of tiles.  Tile rounds in
// lock-step end in synchronized bursts (every CU stores its 128 KB tile, then
// every CU waits for its next tile's first k-tile); here the next tile's first
// k-tile is requested during the current tile's last k-tile, so it is in
// flight while the current tile is stored.  The tiles are dealt per XCD
// (workgroup w runs on XCD w % 8): XCD x owns a contiguous range of tiles, its
// workgroups take them round-robin, so the tiles of one plane, which read the
// same rows, run together on one L2.  (Splitting the tiles left over after
// even rounds into 256 x 128 halves, dealt first to half the workgroups and
// last to the others, measured slower at N = 768: 0.177 vs 0.168 ms.)
#include "common.h"
#include "gemm_nt.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

__global__ __launch_bounds__(kNtThreads) void bgemm_nt_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                              bf16* __restrict__ C, int n, int total, int nwg) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  const int tpr = n / kNtTile, tiles = tpr * tpr;
  const size_t plane = (size_t)n * n;
  // this workgroup's tiles: t = first + l, first + l + L, ... < last
  const int xcd = blockIdx.x % kNtXcds, l = blockIdx.x / kNtXcds, L = nwg / kNtXcds;
  const int per_xcd = (total + kNtXcds - 1) / kNtXcds;
  const int first = xcd * per_xcd, last = min(total, first + per_xcd);
  int t = first + l;
  if (t >= last) return;   // the whole workgroup, before any barrier

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;
  const NtStaging stg(wave, lane, n, kNtTile);
  int offj[4], offi[2];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) offj[jb] = wj * 128 + jb * 32 + perm32(ln);
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) offi[ib] = wi * 64 + ib * 32 + ln;
  const unsigned rows_bytes = (unsigned)kNtTile * n * 2;
  auto a_rsrc = [&](int tt) {
    const int z = tt / tiles, r = tt % tiles;
    return buffer_rsrc(A + z * plane + (size_t)(r / tpr) * kNtTile * n, rows_bytes);
  };
  auto b_rsrc = [&](int tt) {
    const int z = tt / tiles, r = tt % tiles;
    return buffer_rsrc(B + z * plane + (size_t)(r % tpr) * kNtTile * n, rows_bytes);
  };
  const int nk = n / kNtBK;
  __amdgpu_buffer_rsrc_t ra = a_rsrc(t), rb = b_rsrc(t);
  stg.issue(ra, rb, rb, smem, wave, 0);
  int g = 0;   // k-tiles consumed so far: stage g & 1 holds the current one
#pragma unroll 1
  for (; t < last; t += L) {
    const int tn = t + L;
    __amdgpu_buffer_rsrc_t ran = ra, rbn = rb;
    if (tn < last) {
      ran = a_rsrc(tn);
      rbn = b_rsrc(tn);
    }
    f32x16 acc[4][2];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = zero16();
#pragma unroll 1
    for (int kt = 0; kt < nk; ++kt, ++g) {
      __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of the k-tile landed
      __syncthreads();                       // ... and everyone's; the other stage is free again
      bf16* nxt = smem + ((g + 1) & 1) * kNtStage;
      if (kt + 1 < nk)
        stg.issue(ra, rb, rb, nxt, wave, (kt + 1) * kNtBK);
      else if (tn < last)
        stg.issue(ran, rbn, rbn, nxt, wave, 0);   // the next tile's first k-tile
      nt_ktile(smem + (g & 1) * kNtStage, offj, offi, lh, acc);
    }
    // epilogue: plain row-major store of the tile (registers only)
    const int z = t / tiles, rt = t % tiles;
    bf16* Cb = C + z * plane + (size_t)((rt / tpr) * kNtTile) * n + (rt % tpr) * kNtTile;
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
    ra = ran;
    rb = rbn;
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
  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const long long total = batch * (n / kNtTile) * (n / kNtTile);
  // one workgroup per CU (128 KB of LDS each), a multiple of the 8 XCDs, no more than the tiles
  const long long nwg = std::max<long long>(kNtXcds, std::min<long long>(cus, (total + kNtXcds - 1) / kNtXcds * kNtXcds)
                                                         / kNtXcds * kNtXcds);
  KernelTimerScope timed("bgemm_nt", stream);
  hipLaunchKernelGGL(bgemm_nt_kernel, dim3((unsigned)nwg), dim3(kNtThreads), kNtSmem, stream,
                     static_cast<const bf16*>(A), static_cast<const bf16*>(B), static_cast<bf16*>(C), (int)n,
                     (int)total, (int)nwg);
  return check_launch("bgemm_nt");
}

}  // namespace bioemu
