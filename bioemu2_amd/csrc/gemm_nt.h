// One 256 x 256 output tile of C = A B^T on MFMA, A and B row-major with k
// contiguous (an "NT" GEMM), for gfx950.  The tile loop serves the triangle
// contraction (bgemm.hip); the pair-weighted-averaging kernel (pwa.hip)
// reuses its LDS swizzle, staging copy and XCD constants.
//
// Tiling: BK = 64, 512 threads = 8 waves in a 4 (i) x 2 (j) grid, each wave
// 64 (i) x 128 (j) = 2 x 4 MFMA 32x32x16 blocks.  Per 16-deep k-step a wave
// reads 6 operand fragments for 8 MFMAs.  The MFMA A operand is the B tile
// (rows j, permuted with perm32) and the B operand is the A tile (rows i), so
// accumulator acc[jb][ib], lane (ln, lh), register u holds
//   C[i = wi*64 + ib*32 + ln][j = wj*128 + jb*32 + 16 lh + u]
// (16 consecutive j of one i: epilogues write 32-byte runs).
// Global -> LDS staging uses buffer loads with an LDS destination (1 KB per
// instruction, no registers), double-buffered: k-tile kt + 1 is in flight
// while kt is multiplied.  LDS rows are 128 bytes, unpadded, with the 16-byte
// chunk index XOR-swizzled per row.  The k reduction order is fixed (k = 0,
// 1, ... in 16-wide MFMA steps), so appending zero-valued k columns never
// changes a result bit.
#pragma once

#include "common.h"
#include "pairtile.h"

namespace bioemu {

constexpr int kNtTile = 256;                   // BM = BN
constexpr int kNtBK = 64;
constexpr int kNtThreads = 512;
constexpr int kNtTileElems = kNtTile * kNtBK;  // one operand tile: [256 rows][8 chunks of 8]
constexpr int kNtStage = 2 * kNtTileElems;     // A tile | B tile
constexpr int kNtSmem = 2 * kNtStage * 2;      // bytes: double-buffered, 128 KB
constexpr int kNtXcds = 8;

// 16-byte chunk swizzle of a 128-byte tile row: XOR with row bits 1..3.  On
// gfx950 a ds_read_b128 whose 32 lanes read 32 rows of one 32-row block (in
// natural or perm32 order, chunk c or c + 1 per half-wave) is free of bank
// conflicts exactly when the swizzle takes row bit 1 and two of bits 2..4 and
// not row bit 0 (measured with the SQ_LDS_BANK_CONFLICT counter).
__device__ __forceinline__ int nt_swz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int nt_off(int r, int c) { return (r * 8 + (c ^ nt_swz(r))) * 8; }

__device__ __forceinline__ void nt_copy16_to_lds(__amdgpu_buffer_rsrc_t r, const bf16* lds, unsigned voff,
                                                 unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16, voff, soff, 0, 0);
}

// Staging of one operand pair into LDS.  Each operand tile (256 rows x 128 B)
// is 32 copies of 1 KB; wave w moves copies w, w + 8, w + 16, w + 24 of A and
// of B.  Copy j writes LDS chunk 64 j + lane = (row, swizzled chunk) of the
// tile: rows 8 j .. 8 j + 7, all on one side of b_split (B rows [0, b_split)
// from rb, the rest from rb2, whose row 0 is tile row b_split).  Rows are ld
// elements apart.
struct NtStaging {
  unsigned voff[4], voffb[4];
  bool second[4];
  __device__ __forceinline__ NtStaging(int wave, int lane, int ld, int b_split) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int p = (wave + 8 * q) * 64 + lane, r = p >> 3, c = (p & 7) ^ nt_swz(p >> 3);
      voff[q] = (unsigned)(r * ld + c * 8) * 2;
      second[q] = b_split < kNtTile && (wave + 8 * q) * 8 >= b_split;
      voffb[q] = second[q] ? (unsigned)((r - b_split) * ld + c * 8) * 2 : voff[q];
    }
  }
  // k-tile starting at element k0 of every row into stage st (A tile | B tile)
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                        __amdgpu_buffer_rsrc_t rb2, bf16* st, int wave, int k0) const {
    const unsigned soff = (unsigned)k0 * 2;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      nt_copy16_to_lds(ra, st + (wave + 8 * q) * 512, voff[q], soff);
      nt_copy16_to_lds(second[q] ? rb2 : rb, st + kNtTileElems + (wave + 8 * q) * 512, voffb[q], soff);
    }
  }
};

// The 32 MFMAs of one staged k-tile (64 deep) for this wave's 64 x 128 block:
// acc[jb][ib] += B rows (wj*128 + jb*32 + perm32(.)) x A rows (wi*64 + ib*32 + .).
// All 24 operand fragments of the k-tile are requested before the first MFMA
// (the scheduler otherwise recycles a few registers and waits on every read);
// the MFMAs then consume them as they land.
__device__ __forceinline__ void nt_ktile(const bf16* st, const int (&offj)[4], const int (&offi)[2], int lh,
                                         f32x16 (&acc)[4][2]) {
  const bf16* sa = st;
  const bf16* sb = st + kNtTileElems;
  bf16x8 fj[4][4], fi[4][2];
#pragma unroll
  for (int ks = 0; ks < kNtBK / 16; ++ks) {
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) fj[ks][jb] = load8(sb + nt_off(offj[jb], 2 * ks + lh));
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) fi[ks][ib] = load8(sa + nt_off(offi[ib], 2 * ks + lh));
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ks = 0; ks < kNtBK / 16; ++ks)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = mfma32(fj[ks][jb], fi[ks][ib], acc[jb][ib]);
  __builtin_amdgcn_sched_barrier(0);
}

// A points at the tile's first row of A, of which a_rows (<= 256) exist: the
// rest read as zero through the buffer bound (their C rows are garbage-free
// zeros times B, never needed by a caller that skips them).  B rows [0,
// b_split) come from B, rows [b_split, 256) from B2 (its row 0 = tile row
// b_split), of which b2_rows exist (rows past them read as zero through the
// buffer bound); b_split is a multiple of 8.  Rows are ld elements apart, of which
// the first K (K % 64 == 0, K <= ld) are reduced; 256 * ld * 2 < 2^32.  Whole
// workgroup; smem holds kNtSmem bytes.  Ends with an epilogue-ready acc and no
// copy in flight; other waves may still read the last stage (an epilogue that
// reuses smem starts with a barrier).
__device__ __forceinline__ void gemm_nt_tile(const bf16* A, int a_rows, const bf16* B, const bf16* B2, int b_split,
                                             int b2_rows, int K, int ld, bf16* smem, f32x16 (&acc)[4][2]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A, (unsigned)a_rows * ld * 2);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B, (unsigned)b_split * ld * 2);
  const __amdgpu_buffer_rsrc_t rb2 = buffer_rsrc(B2, (unsigned)min(kNtTile - b_split, b2_rows) * ld * 2);
  const NtStaging stg(wave, lane, ld, b_split);

#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) acc[jb][ib] = zero16();

  const int nk = K / kNtBK;
  stg.issue(ra, rb, rb2, smem, wave, 0);
  int offj[4], offi[2];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) offj[jb] = wj * 128 + jb * 32 + perm32(ln);
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) offi[ib] = wi * 64 + ib * 32 + ln;
#pragma unroll 1
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of k-tile kt landed
    __syncthreads();                       // ... and everyone's; the other stage is free again
    if (kt + 1 < nk) stg.issue(ra, rb, rb2, smem + ((kt + 1) & 1) * kNtStage, wave, (kt + 1) * kNtBK);
    nt_ktile(smem + (kt & 1) * kNtStage, offj, offi, lh, acc);
  }
}

// Full tiles from one B matrix.
__device__ __forceinline__ void gemm_nt_tile(const bf16* A, const bf16* B, int K, bf16* smem, f32x16 (&acc)[4][2]) {
  gemm_nt_tile(A, kNtTile, B, B, kNtTile, 0, K, K, smem, acc);
}

// XCD-aware work-item order: workgroup w runs on XCD w % 8; each XCD gets a
// contiguous range of items (so the tiles of one plane share its L2).
// grid = items rounded up to a multiple of 8; returns -1 for padding groups.
__device__ __forceinline__ int nt_item(int total) {
  const int w = blockIdx.x;
  const int per_xcd = (total + kNtXcds - 1) / kNtXcds;
  const int item = (w % kNtXcds) * per_xcd + w / kNtXcds;
  return item < total ? item : -1;
}

}  // namespace bioemu
