// Batched bf16 NT GEMM on MFMA: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k].
//
// Used for the per-channel triangle contraction, where both operands are
// channel-major [z = b*D + d][row][k] planes with k contiguous.  M = N = K = n,
// n a multiple of 256, so the kernel has no edge handling; callers zero-pad.
//
// Tiling: 256 x 256 workgroup tile, BK = 64, 512 threads = 8 waves in a
// 4 (i) x 2 (j) grid, each wave 64 (i) x 128 (j) = 2 x 4 MFMA 32x32x16 blocks.
// Per 16-deep k-step a wave reads 6 operand fragments for 8 MFMAs.  The MFMA
// A operand is the B tile (rows j, permuted with perm32) and the B operand is
// the A tile (rows i), so an accumulator lane holds 16 consecutive j of one i:
// C rows are written as 32-byte runs straight from registers.
// Global -> LDS staging uses buffer loads with an LDS destination (1 KB per
// instruction, no registers), double-buffered: k-tile kt + 1 is in flight
// while kt is multiplied.  LDS rows are 128 bytes, unpadded, with the 16-byte
// chunk index XOR-swizzled per row.  The k reduction order is fixed (k = 0,
// 1, ... in 16-wide MFMA steps), so appending zero-valued k columns never
// changes a result bit.
//
// Workgroup -> (plane, tile) mapping is XCD-aware: consecutive workgroup ids
// are dispatched round-robin over the 8 XCDs, so ids are regrouped such that
// all tiles of one plane land on one XCD and share its L2.
#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kThreads = 512;
constexpr int kTileElems = BM * BK;           // one operand tile: [256 rows][8 chunks of 8]
constexpr int kStage = 2 * kTileElems;        // A tile | B tile
constexpr int kSmem = 2 * kStage * 2;         // bytes: double-buffered, 128 KB
constexpr int kXcds = 8;

// 16-byte chunk swizzle of a 128-byte tile row: conflict-free both for rows
// read in natural order and in perm32 order (16 lanes -> 16 bank groups).
__device__ __forceinline__ int swz(int r) { return ((r >> 1) & 7) ^ (((r >> 4) & 1) << 2); }
__device__ __forceinline__ int t_off(int r, int c) { return (r * 8 + (c ^ swz(r))) * 8; }

__device__ __forceinline__ void copy16_to_lds(__amdgpu_buffer_rsrc_t r, const bf16* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16, voff, soff, 0, 0);
}

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
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;

  const size_t plane = (size_t)n * n;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A + z * plane + (size_t)ti * BM * n, (unsigned)BM * n * 2);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B + z * plane + (size_t)tj * BN * n, (unsigned)BN * n * 2);
  // Staging: each operand tile (256 rows x 128 B) is 32 copies of 1 KB; wave w
  // moves copies w, w + 8, w + 16, w + 24 of A and of B.  Copy j writes LDS
  // chunk 64 j + lane = (row, swizzled chunk) of the tile.
  unsigned voff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int p = (wave + 8 * q) * 64 + lane, r = p >> 3, c = (p & 7) ^ swz(p >> 3);
    voff[q] = (unsigned)(r * n + c * 8) * 2;
  }
  auto stage = [&](int kt) {
    bf16* st = smem + (kt & 1) * kStage;
    const unsigned soff = (unsigned)(kt * BK) * 2;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      copy16_to_lds(ra, st + (wave + 8 * q) * 512, voff[q], soff);
      copy16_to_lds(rb, st + kTileElems + (wave + 8 * q) * 512, voff[q], soff);
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = zero16();

  const int nk = n / BK;
  stage(0);
  const int jrow = perm32(ln);
#pragma unroll 1
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of k-tile kt landed
    __syncthreads();                       // ... and everyone's; the other stage is free again
    if (kt + 1 < nk) stage(kt + 1);
    const bf16* sa = smem + (kt & 1) * kStage;
    const bf16* sb = sa + kTileElems;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8 fj[4], fi[2];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) fj[jb] = load8(sb + t_off(wj * 128 + jb * 32 + jrow, 2 * ks + lh));
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) fi[ib] = load8(sa + t_off(wi * 64 + ib * 32 + ln, 2 * ks + lh));
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = mfma32(fj[jb], fi[ib], acc[jb][ib]);
    }
  }

  // D lane (ln, lh) of block (jb, ib): i = wi*64 + ib*32 + ln, j = wj*128 + jb*32 + 16lh + u.
  bf16* Cb = C + z * plane + (size_t)(ti * BM) * n + tj * BN;
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
  if (n % kGemmTile != 0 || n <= 0 || batch <= 0 || batch * (n / BM) * (n / BN) > (1ll << 31) - 1 ||
      (long long)BM * n * 2 > 0xffffffffLL) {
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
