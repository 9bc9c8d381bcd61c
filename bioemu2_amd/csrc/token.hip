// Token-side (single representation) kernels for gfx950: row LayerNorm, a
// small MFMA GEMM with fused epilogues, and two GEMMs on the LDS-staged
// 256 x 256 tile loop of gemm_nt.h.  These carry the per-token parts of
// AttentionPairBias (src/bioemu2/biomoa/ops/attention_pair_bias.py:150-161,
// :224-225), of the sliding-window attention, and the single-representation
// Transition (src/bioemu2/biomoa/ops/transition.py:52-91).  In the trunk the
// token dimension is small (B * N rows of c_s = 384): there one wave computes
// one 32x32 output block with operands read straight from L2
// (token_gemm_kernel).  The denoiser's copies make it large (M = 8 copies of
// 768 tokens, 8 x 6144 atoms): the attention's four input projections always
// run as one tiled launch (token_qkvg_kernel) and its output projection takes
// the tiled kernel above a measured size (token_out_kernel).
//
// Row spaces.  A GEMM runs over M = B * Np "padded" rows (Np = N rounded up to
// 32, rows t >= N of each batch are zero).  Row-major outputs/residuals use
// either the same padded layout or, with out_rows = N, the caller's compact
// [B][N] layout (padded rows are then dropped).  Transposed outputs are laid
// out [B][Nout][Np].
#include "common.h"
#include "gemm_nt.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

enum Epilogue : int {
  kEpiStore = 0,     // out = acc (+ col_bias)
  kEpiSigmoid = 1,   // out = sigmoid(acc)
  kEpiSwiGLU = 2,    // out = silu(A W^T) * (A W2^T)
  kEpiResidual = 3,  // out = res + acc
};

// ---------------------------------------------------------------------------
// y[b][t] = LN(x[b][t]) for t < N, 0 for N <= t < Np.  One wave per row,
// K <= 512 and K % 64 == 0 (each lane holds K/64 values).  gamma == null
// copies the rows unnormalised (same padding).
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(256) void token_ln_kernel(const bf16* __restrict__ x, const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, bf16* __restrict__ y, int B,
                                                       int N, int Np, float eps) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (long long)B * Np) return;
  const int b = (int)(row / Np), t = (int)(row % Np);
  constexpr int PER = K / 64;
  bf16* yr = y + (size_t)row * K;
  if (t >= N) {
#pragma unroll
    for (int e = 0; e < PER; ++e) yr[lane + 64 * e] = f2bf(0.f);
    return;
  }
  const bf16* xr = x + ((size_t)b * N + t) * K;
  float v[PER];
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    v[e] = bf2f(xr[lane + 64 * e]);
    s += v[e];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  const float mean = s * (1.0f / K);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const float d = v[e] - mean;
    ss += d * d;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float rstd = rsqrtf(ss * (1.0f / K) + eps);
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int c = lane + 64 * e;
    float o = v[e];
    if (gamma) {
      o = (v[e] - mean) * rstd * gamma[c];
      if (beta) o += beta[c];
    }
    yr[c] = f2bf(o);
  }
}

// Any width K (a runtime loop over this lane's channels lane, lane + 64, ...):
// the same rows and padding as token_ln_kernel, for widths outside its
// compile-time set (the denoiser's token/atom mixers, dim = a_s + atom_s).
__global__ __launch_bounds__(256) void token_ln_any_kernel(const bf16* __restrict__ x, const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, bf16* __restrict__ y, int B,
                                                           int N, int Np, int K, float eps) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (long long)B * Np) return;
  const int b = (int)(row / Np), t = (int)(row % Np);
  bf16* yr = y + (size_t)row * K;
  if (t >= N) {
    for (int c = lane; c < K; c += 64) yr[c] = f2bf(0.f);
    return;
  }
  const bf16* xr = x + ((size_t)b * N + t) * K;
  float s = 0.f;
  for (int c = lane; c < K; c += 64) s += bf2f(xr[c]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  const float mean = s / (float)K;
  float ss = 0.f;
  for (int c = lane; c < K; c += 64) {
    const float d = bf2f(xr[c]) - mean;
    ss += d * d;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float rstd = rsqrtf(ss / (float)K + eps);
  for (int c = lane; c < K; c += 64) {
    float o = bf2f(xr[c]);
    if (gamma) {
      o = (o - mean) * rstd * gamma[c];
      if (beta) o += beta[c];
    }
    yr[c] = f2bf(o);
  }
}

// ---------------------------------------------------------------------------
// out = epilogue(A[M][K] * W[Nout][K]^T) on 32x32 output blocks, 4 waves per
// workgroup.  The token GEMMs are skinny (a few hundred rows), so for K >= 256
// the k reduction of a block is split over the workgroup's 4 waves (wave w
// takes the 16-deep steps k = 16 w, 16 (w + 4), ...): 4x the workgroups in
// flight and a quarter of each wave's chain of dependent loads; wave 0 adds
// the other waves' partial sums in a fixed order (deterministic) and runs the
// epilogue.  For smaller K each wave owns a block of its own.
// Row-major (kTrans = false): D = W A^T, lane (n, hh) holds row n and columns
// 16hh..16hh+15 of the block.  Transposed (kTrans = true): D = A W^T with A
// rows permuted, lane (n, hh) holds column n and rows 16hh..16hh+15.
// ---------------------------------------------------------------------------
constexpr int kSplitK = 4;        // most waves per workgroup
constexpr int kSplitMinK = 256;   // smaller K: one wave, no reduction

template <int kEpi, bool kTrans>
__global__ __launch_bounds__(64 * kSplitK) void token_gemm_kernel(const bf16* __restrict__ A,
                                                                  const bf16* __restrict__ W,
                                                                  const bf16* __restrict__ W2,
                                                                  const float* __restrict__ col_bias,
                                                                  const bf16* res, bf16* out, int8_t* tail, int M,
                                                                  int K, int Nout, int N, int Np, int out_rows) {
  constexpr int kAccs = kEpi == kEpiSwiGLU ? 2 : 1;
  __shared__ float part[kSplitK - 1][kAccs][16][64];   // partial sums of waves 1..3, lane-contiguous
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int splits = K >= kSplitMinK ? kSplitK : 1;   // waves per block (uniform)
  const int kw = wave % splits;                        // this wave's share of the k steps
  const int blk = blockIdx.x * (kSplitK / splits) + wave / splits;
  const int nb = Nout / 32;
  if (blk >= ((M + 31) / 32) * nb) return;   // only when splits == 1: no barrier follows
  const int row0 = (blk / nb) * 32, col0 = (blk % nb) * 32;
  const int n = lane & 31, hh = lane >> 5;

  f32x16 acc = zero16(), acc2 = zero16();
  if (!kTrans) {
    const bf16* wr = W + (size_t)(col0 + perm32(n)) * K + 8 * hh;
    const bf16* wr2 = (kEpi == kEpiSwiGLU) ? W2 + (size_t)(col0 + perm32(n)) * K + 8 * hh : nullptr;
    const int ra = min(row0 + n, M - 1);
    const bf16* ar = A + (size_t)ra * K + 8 * hh;
    for (int k = 16 * kw; k < K; k += 16 * splits) {
      const bf16x8 af = load8(ar + k);
      acc = mfma32(load8(wr + k), af, acc);
      if (kEpi == kEpiSwiGLU) acc2 = mfma32(load8(wr2 + k), af, acc2);
    }
  } else {
    const int ra = min(row0 + perm32(n), M - 1);
    const bf16* ar = A + (size_t)ra * K + 8 * hh;
    const bf16* wr = W + (size_t)(col0 + n) * K + 8 * hh;
    for (int k = 16 * kw; k < K; k += 16 * splits) acc = mfma32(load8(ar + k), load8(wr + k), acc);
  }
  if (splits > 1) {   // workgroup-uniform
    if (wave > 0) {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        part[wave - 1][0][u][lane] = acc[u];
        if (kEpi == kEpiSwiGLU) part[wave - 1][kAccs - 1][u][lane] = acc2[u];
      }
    }
    __syncthreads();
    if (wave > 0) return;   // after the only barrier
    for (int q = 0; q < splits - 1; ++q)
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        acc[u] += part[q][0][u][lane];
        if (kEpi == kEpiSwiGLU) acc2[u] += part[q][kAccs - 1][u][lane];
      }
  }

  float v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    float a = acc[u];
    if (kEpi == kEpiSigmoid) a = sigmoidf_fast(a);
    if (kEpi == kEpiSwiGLU) a = siluf_fast(a) * acc2[u];
    v[u] = a;
  }

  if (!kTrans) {
    const int r = row0 + n;
    if (r >= M) return;
    const int b = r / Np, t = r % Np;
    if (out_rows != Np && t >= out_rows) return;
    const size_t orow = (out_rows == Np) ? (size_t)r : (size_t)b * out_rows + t;
    const int c0 = col0 + 16 * hh;
    if (kEpi == kEpiStore && col_bias) {
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] += col_bias[c0 + u];
    }
    if (kEpi == kEpiResidual && tail) {   // residual stream with an int8 tail (common.h), in place
      float rv[16];
      tail_decode16(load8(res + orow * Nout + c0), load8(res + orow * Nout + c0 + 8),
                    load_tail16(tail + orow * Nout + c0), rv);
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] += rv[u];
      tail_store16(out + orow * Nout + c0, tail + orow * Nout + c0, v);
      return;
    }
    if (kEpi == kEpiResidual) {
      const bf16x8 r0 = load8(res + orow * Nout + c0), r1 = load8(res + orow * Nout + c0 + 8);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        v[u] += bf2f(r0[u]);
        v[8 + u] += bf2f(r1[u]);
      }
    }
    store16(out + orow * Nout + c0, v);
  } else {
    // rows row0 + 16hh .. +15 of column col0 + n; a 16-row run never crosses a batch (Np % 32 == 0)
    const int r = row0 + 16 * hh;
    if (r >= M) return;
    const int b = r / Np, t = r % Np;
    store16(out + ((size_t)b * Nout + col0 + n) * Np + t, v);
  }
}

// ---------------------------------------------------------------------------
// q | k | v^T | g of an attention in one launch: 256 x 256 tiles of
// sn[M][c_s] times [Wq; Wk; Wv; Wg]^T ([4 c_s][c_s], weights staged through
// LDS by the tile loop of gemm_nt.h; tile rows past M read as zero and are not
// stored).  The output is picked per 32-column block: q ((+ q_bias) * q_scale),
// k and g (sigmoid) row-major [M][c_s]; v transposed per sequence of
// seq_rows rows, [M / seq_rows][c_s][seq_rows] (row r = sequence r / seq_rows,
// position r % seq_rows).  Lane (ln, lh) of block (ib, jb) holds row
// wi*64 + ib*32 + ln and 16 consecutive output columns (gemm_nt.h).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNtThreads) void token_qkvg_kernel(const bf16* __restrict__ sn,
                                                                const bf16* __restrict__ wqkv,
                                                                const bf16* __restrict__ wg,
                                                                const float* __restrict__ q_bias, float q_scale,
                                                                bf16* __restrict__ q, bf16* __restrict__ k,
                                                                bf16* __restrict__ vt, bf16* __restrict__ g, int M,
                                                                int CS, int seq_rows) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  const int ntj = 4 * CS / kNtTile;
  const int ti = blockIdx.x / ntj, tj = blockIdx.x % ntj;
  const int row0 = ti * kNtTile, col0 = tj * kNtTile;
  // weight rows col0 .. col0 + 255: [0, 3 c_s) are wqkv's, [3 c_s, 4 c_s) wg's
  const int split = min(max(3 * CS - col0, 0), kNtTile);
  const bf16* b1 = wqkv + (size_t)min(col0, 3 * CS) * CS;
  const bf16* b2 = wg + (size_t)max(col0 - 3 * CS, 0) * CS;
  f32x16 acc[4][2];
  gemm_nt_tile(sn + (size_t)row0 * CS, min(M - row0, kNtTile), b1, b2, split, CS - max(col0 - 3 * CS, 0), CS, CS,
               smem, acc);

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    const int col = col0 + wj * 128 + jb * 32;   // wave-uniform 32-column block
    const int which = col / CS, c0 = col % CS + 16 * lh;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int r = row0 + wi * 64 + ib * 32 + ln;
      if (r >= M) continue;
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = acc[jb][ib][u];
      if (which == 2) {
        const int sq = r / seq_rows, t = r % seq_rows;
        bf16* dst = vt + ((size_t)sq * CS + c0) * seq_rows + t;
#pragma unroll
        for (int u = 0; u < 16; ++u) dst[(size_t)u * seq_rows] = f2bf(v[u]);
        continue;
      }
      if (which == 0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = (v[u] + q_bias[c0 + u]) * q_scale;
      } else if (which == 3) {
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = sigmoidf_fast(v[u]);
      }
      store16((which == 0 ? q : which == 1 ? k : g) + (size_t)r * CS + c0, v);
    }
  }
}

// ---------------------------------------------------------------------------
// out = A[M][K] W[Nout][K]^T (+ res) on 256 x 256 tiles (gemm_nt.h tile loop,
// operands staged through LDS; rows past M read as zero, columns past Nout
// are computed on W's rows from row 0 again, or zeros past W's end, and are
// not stored).  Rows are batches of
// Np padded rows; with out_rows < Np the output / residual use the compact
// [B][out_rows] layout and padded rows are dropped (as token_gemm_kernel).
// With a tail (kTail) the residual stream carries int8 tails, in place.
// ---------------------------------------------------------------------------
template <bool kResidual, bool kTail>
__global__ __launch_bounds__(kNtThreads) void token_out_kernel(const bf16* __restrict__ A, const bf16* __restrict__ W,
                                                               const bf16* res, bf16* out, int8_t* tail, int M, int K,
                                                               int Nout, int Np, int out_rows) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  const int ntj = (Nout + kNtTile - 1) / kNtTile;
  const int ti = blockIdx.x / ntj, tj = blockIdx.x % ntj;
  const int row0 = ti * kNtTile, col0 = tj * kNtTile;
  const int valid_cols = min(Nout - col0, kNtTile);   // a multiple of 32
  f32x16 acc[4][2];
  // columns past Nout take W's rows from row 0 again (W has Nout rows; the
  // rest of the tile reads as zero) and are not stored
  gemm_nt_tile(A + (size_t)row0 * K, min(M - row0, kNtTile), W + (size_t)col0 * K, W, valid_cols, Nout, K, K, smem,
               acc);

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 3, wj = wave >> 2;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    const int cl = wj * 128 + jb * 32;   // wave-uniform 32-column block of the tile
    if (cl >= valid_cols) continue;
    const int c0 = col0 + cl + 16 * lh;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int r = row0 + wi * 64 + ib * 32 + ln;
      if (r >= M) continue;
      const int b = r / Np, t = r % Np;
      if (t >= out_rows) continue;
      const size_t off = ((size_t)b * out_rows + t) * Nout + c0;
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = acc[jb][ib][u];
      if (kTail) {
        float rv[16];
        tail_decode16(load8(res + off), load8(res + off + 8), load_tail16(tail + off), rv);
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] += rv[u];
        tail_store16(out + off, tail + off, v);
        continue;
      }
      if (kResidual) {
        const bf16x8 r0 = load8(res + off), r1 = load8(res + off + 8);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          v[u] += bf2f(r0[u]);
          v[8 + u] += bf2f(r1[u]);
        }
      }
      store16(out + off, v);
    }
  }
}

template <int kEpi, bool kTrans>
int launch_gemm(const void* A, const void* W, const void* W2, const float* col_bias, const void* res, void* out,
                int8_t* tail, int64_t M, int64_t K, int64_t Nout, int64_t N, int64_t Np, int64_t out_rows,
                hipStream_t stream, const char* name) {
  const int64_t blocks = ((M + 31) / 32) * (Nout / 32);
  const int64_t per_wg = K >= kSplitMinK ? 1 : kSplitK;   // blocks per workgroup
  KernelTimerScope timed(name, stream);
  hipLaunchKernelGGL((token_gemm_kernel<kEpi, kTrans>), dim3((unsigned)((blocks + per_wg - 1) / per_wg)),
                     dim3(64 * kSplitK), 0, stream,
                     static_cast<const bf16*>(A), static_cast<const bf16*>(W), static_cast<const bf16*>(W2),
                     col_bias, static_cast<const bf16*>(res), static_cast<bf16*>(out), tail, (int)M, (int)K, (int)Nout,
                     (int)N, (int)Np, (int)out_rows);
  return check_launch(name);
}

}  // namespace

int token_layernorm(const void* x, const float* gamma, const float* beta, void* y, int64_t B, int64_t N,
                    int64_t Np, int64_t K, hipStream_t stream) {
  const int64_t rows = B * Np;
  dim3 grid((unsigned)((rows + 3) / 4));
  KernelTimerScope timed("token_layernorm", stream);
  switch (K) {
    case 64:
      hipLaunchKernelGGL(token_ln_kernel<64>, grid, dim3(256), 0, stream, static_cast<const bf16*>(x), gamma, beta,
                         static_cast<bf16*>(y), (int)B, (int)N, (int)Np, 1e-5f);
      break;
    case 128:
      hipLaunchKernelGGL(token_ln_kernel<128>, grid, dim3(256), 0, stream, static_cast<const bf16*>(x), gamma, beta,
                         static_cast<bf16*>(y), (int)B, (int)N, (int)Np, 1e-5f);
      break;
    case 384:
      hipLaunchKernelGGL(token_ln_kernel<384>, grid, dim3(256), 0, stream, static_cast<const bf16*>(x), gamma, beta,
                         static_cast<bf16*>(y), (int)B, (int)N, (int)Np, 1e-5f);
      break;
    default:
      if (K <= 0) return set_error(BIOEMU_ERR_UNSUPPORTED, "token_layernorm: width %lld unsupported", (long long)K);
      hipLaunchKernelGGL(token_ln_any_kernel, grid, dim3(256), 0, stream, static_cast<const bf16*>(x), gamma, beta,
                         static_cast<bf16*>(y), (int)B, (int)N, (int)Np, (int)K, 1e-5f);
  }
  return check_launch("token_layernorm");
}

int token_gemm(int epi, bool trans, const void* A, const void* W, const void* W2, const float* col_bias,
               const void* res, void* out, int64_t M, int64_t K, int64_t Nout, int64_t N, int64_t Np,
               int64_t out_rows, hipStream_t stream, const char* name, int8_t* tail) {
  if (M <= 0 || K <= 0 || K % 16 || Nout <= 0 || Nout % 32 || Np % 32 || M % Np)
    return set_error(BIOEMU_ERR_INVALID_ARG, "%s: bad GEMM shape M=%lld K=%lld Nout=%lld Np=%lld", name,
                     (long long)M, (long long)K, (long long)Nout, (long long)Np);
  if (tail && (epi != kEpiResidual || trans))
    return set_error(BIOEMU_ERR_INVALID_ARG, "%s: a residual tail needs the residual epilogue", name);
  if (trans) {
    if (epi != kEpiStore) return set_error(BIOEMU_ERR_INVALID_ARG, "%s: transposed GEMM stores plainly", name);
    return launch_gemm<kEpiStore, true>(A, W, W2, col_bias, res, out, tail, M, K, Nout, N, Np, out_rows, stream, name);
  }
  switch (epi) {
    case kEpiStore:
      return launch_gemm<kEpiStore, false>(A, W, W2, col_bias, res, out, tail, M, K, Nout, N, Np, out_rows, stream, name);
    case kEpiSigmoid:
      return launch_gemm<kEpiSigmoid, false>(A, W, W2, col_bias, res, out, tail, M, K, Nout, N, Np, out_rows, stream, name);
    case kEpiSwiGLU:
      return launch_gemm<kEpiSwiGLU, false>(A, W, W2, col_bias, res, out, tail, M, K, Nout, N, Np, out_rows, stream, name);
    case kEpiResidual:
      return launch_gemm<kEpiResidual, false>(A, W, W2, col_bias, res, out, tail, M, K, Nout, N, Np, out_rows, stream, name);
    default:
      return set_error(BIOEMU_ERR_INVALID_ARG, "%s: unknown epilogue %d", name, epi);
  }
}


int token_qkvg(const void* sn, const void* wqkv, const void* w_g, const float* q_bias, float q_scale, void* q,
               void* k, void* vt, void* g, int64_t M, int64_t CS, int64_t seq_rows, hipStream_t stream,
               const char* name) {
  if (M <= 0 || CS <= 0 || CS % 64 || seq_rows <= 0 || M % seq_rows || M > 0x7fffffffLL ||
      (long long)kNtTile * CS * 2 > 0xffffffffLL)
    return set_error(BIOEMU_ERR_INVALID_ARG, "%s: bad shape M=%lld c_s=%lld rows per sequence=%lld", name,
                     (long long)M, (long long)CS, (long long)seq_rows);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(token_qkvg_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          kNtSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "%s: cannot set dynamic LDS size", name);
  const long long tiles = (M + kNtTile - 1) / kNtTile * (4 * CS / kNtTile);
  KernelTimerScope timed(name, stream);
  hipLaunchKernelGGL(token_qkvg_kernel, dim3((unsigned)tiles), dim3(kNtThreads), kNtSmem, stream,
                     static_cast<const bf16*>(sn), static_cast<const bf16*>(wqkv), static_cast<const bf16*>(w_g), q_bias,
                     q_scale, static_cast<bf16*>(q), static_cast<bf16*>(k), static_cast<bf16*>(vt),
                     static_cast<bf16*>(g), (int)M, (int)CS, (int)seq_rows);
  return check_launch(name);
}


constexpr long long kTiledMinOutputs = 2000000;

int token_out_proj(const void* A, const void* W, const void* res, void* out, int8_t* tail, int64_t M, int64_t K,
                   int64_t Nout, int64_t Np, int64_t out_rows, bool residual, hipStream_t stream, const char* name) {
  if (M <= 0 || K <= 0 || K % 64 || Nout <= 0 || Nout % 32 || Np <= 0 || Np % 32 || M % Np || out_rows > Np ||
      M > 0x7fffffffLL || (long long)kNtTile * K * 2 > 0xffffffffLL)
    return set_error(BIOEMU_ERR_INVALID_ARG, "%s: bad shape M=%lld K=%lld Nout=%lld Np=%lld", name, (long long)M,
                     (long long)K, (long long)Nout, (long long)Np);
  if (tail && !residual) return set_error(BIOEMU_ERR_INVALID_ARG, "%s: a residual tail needs residual=1", name);
  // A 256 x 256 tile takes about as long as the per-block GEMM needs for ~2M
  // outputs (measured: 0.016 vs 0.020 ms at M = 6144, c_s = 384; 0.018 vs
  // 0.015 ms at M = 4096; slower still at M = 768): fewer outputs take the
  // per-block kernel.
  if (M * Nout < kTiledMinOutputs)
    return token_gemm(residual ? kEpiResidualId : kEpiStoreId, false, A, W, nullptr, nullptr, res, out, M, K, Nout,
                      out_rows, Np, out_rows, stream, name, tail);
  const void* k = tail ? reinterpret_cast<const void*>(token_out_kernel<true, true>)
                       : residual ? reinterpret_cast<const void*>(token_out_kernel<true, false>)
                                  : reinterpret_cast<const void*>(token_out_kernel<false, false>);
  if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kNtSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "%s: cannot set dynamic LDS size", name);
  const long long tiles = (M + kNtTile - 1) / kNtTile * ((Nout + kNtTile - 1) / kNtTile);
  KernelTimerScope timed(name, stream);
  const bf16* a = static_cast<const bf16*>(A);
  const bf16* w = static_cast<const bf16*>(W);
  const bf16* r = static_cast<const bf16*>(res);
  bf16* o = static_cast<bf16*>(out);
  if (tail)
    hipLaunchKernelGGL((token_out_kernel<true, true>), dim3((unsigned)tiles), dim3(kNtThreads), kNtSmem, stream, a, w,
                       r, o, tail, (int)M, (int)K, (int)Nout, (int)Np, (int)out_rows);
  else if (residual)
    hipLaunchKernelGGL((token_out_kernel<true, false>), dim3((unsigned)tiles), dim3(kNtThreads), kNtSmem, stream, a,
                       w, r, o, nullptr, (int)M, (int)K, (int)Nout, (int)Np, (int)out_rows);
  else
    hipLaunchKernelGGL((token_out_kernel<false, false>), dim3((unsigned)tiles), dim3(kNtThreads), kNtSmem, stream, a,
                       w, r, o, nullptr, (int)M, (int)K, (int)Nout, (int)Np, (int)out_rows);
  return check_launch(name);
}

}  // namespace bioemu

using namespace bioemu;

// ---------------------------------------------------------------------------
// Single-representation Transition: s (+)= fc3(silu(fc1(LN s)) * fc2(LN s)).
// ---------------------------------------------------------------------------
extern "C" size_t bioemu_transition_token_workspace_bytes(int64_t M, int64_t Dc, int64_t hidden) {
  if (M <= 0 || Dc <= 0 || hidden <= 0) return 0;
  const size_t Mp = (size_t)round_up(M, 32);
  return round_up(Mp * Dc * 2, 256) + round_up(Mp * hidden * 2, 256);
}

extern "C" int bioemu_transition_token_fwd(const void* x, const float* norm_w, const float* norm_b,
                                           const void* fc1_w, const void* fc2_w, const void* fc3_w, void* out,
                                           int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t M,
                                           int64_t Dc, int64_t hidden, int64_t out_dim, int use_norm, int residual,
                                           hipStream_t stream) {
  if (M <= 0 || Dc <= 0 || Dc % 16 || hidden <= 0 || hidden % 32 || out_dim <= 0 || out_dim % 32)
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "transition_token: dim %lld / hidden %lld / out_dim %lld unsupported (dim a multiple of 16, "
                     "hidden and out_dim multiples of 32)", (long long)Dc, (long long)hidden, (long long)out_dim);
  if (residual && out_dim != Dc)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_token: residual=1 needs out_dim == dim");
  if (!x || !fc1_w || !fc2_w || !fc3_w || !out || !workspace || (use_norm && !norm_w))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_token: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(fc1_w) || !aligned16(fc2_w) || !aligned16(fc3_w) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_token: tensors must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_token: out may alias x only with residual=1");
  if (res_tail && (!residual || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_token: res_tail needs residual=1 and 16-byte alignment");
  if (workspace_bytes < bioemu_transition_token_workspace_bytes(M, Dc, hidden))
    return set_error(BIOEMU_ERR_WORKSPACE, "transition_token: workspace too small");
  // Rows are treated as one batch of M tokens padded to Mp.
  const int64_t Mp = round_up(M, 32);
  char* p = static_cast<char*>(workspace);
  bf16* xn = reinterpret_cast<bf16*>(p);
  bf16* hbuf = reinterpret_cast<bf16*>(p + round_up(Mp * Dc * 2, 256));
  int rc = token_layernorm(x, use_norm ? norm_w : nullptr, use_norm ? norm_b : nullptr, xn, 1, M, Mp, Dc, stream);
  if (rc) return rc;
  rc = token_gemm(kEpiSwiGLU, false, xn, fc1_w, fc2_w, nullptr, nullptr, hbuf, Mp, Dc, hidden, M, Mp, Mp, stream,
                  "transition_token_swiglu");
  if (rc) return rc;
  return token_gemm(residual ? kEpiResidual : kEpiStore, false, hbuf, fc3_w, nullptr, nullptr, x, out, Mp, hidden,
                    out_dim, M, Mp, M, stream, "transition_token_out", res_tail);
}
