// Pair-weighted averaging (MSA module) for gfx950.
//
// Reference: PairWeightedAveraging.forward, unchunked path
// (src/bioemu2/biomoa/ops/pair_weighted_averaging.py:125-154), with the widths
// the reference trunk uses (PairMixerMSALayer, biomoa/modules/pairmixer.py:673-678):
// c_m = 64, c_z = 128, c_h = 32, H = 8.
//   m' = LN_m(m);  v = m' Wm^T (heads of 32);  g = sigmoid(m' Wg^T)
//   w[h, i, :] = softmax_j( LN_z(z[i, j]) Wz^T [h], masked keys replaced by -1e6 )
//   o[s, i, h, :] = sum_j w[h, i, j] v[s, j, h, :];   out = (g * o) Wo^T  (+ m)
// The weights do not depend on the MSA row s, so for each head the averaging
// is one GEMM: O_h[i][(s, d)] = sum_j W_h[i][j] V_h^T[(s, d)][j].
//
// Kernels:
//   pwa_weights  : one workgroup per (b, row i): LN_z folded into Wz (MFMA),
//                  the 8 logit rows in LDS, masked, softmax over j -> W bf16.
//   pwa_proj     : LN_m folded into Wm | Wg; per 32 tokens of one MSA row the
//                  v block comes out channel-major (V^T, j contiguous: the
//                  GEMM's B operand) and g pair-major.
//   pwa_fused    : per head the averaging GEMM on MFMA, then the gate and
//                  the output projection from the accumulator registers;
//                  writes (g * o) Wo^T (+ m) once, after the last head.
// Padding: tokens are padded to Np = N rounded up to 256 (GEMM tiles), MSA rows
// to S8 = S rounded up to 8; padded keys have weight exactly 0 and padded v
// rows are exactly 0, so padding never changes a valid output bit.
#include <algorithm>

#include "common.h"
#include "gemm_nt.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int CM = 64;
constexpr int CZ = 128;
constexpr int CH = 32;
constexpr int NH = 8;
constexpr int HC = NH * CH;   // 256
constexpr int kLdw64 = CM + 8;

// ---------------------------------------------------------------------------
// Weights: grid = B * Np rows, 256 threads.  LDS: folded Wz rows (8, padded to
// a 32-row MFMA block), their bias pairs, then the logits [8][Np] (fp32).
// ---------------------------------------------------------------------------
constexpr int kWThreads = 256;
constexpr int kWFixedSmem = 32 * kLdw * 2 + 32 * 2 * 2;

__global__ __launch_bounds__(kWThreads) void pwa_weights_kernel(const bf16* __restrict__ z,
                                                                const uint8_t* __restrict__ mask,
                                                                const bf16* __restrict__ wzf,
                                                                const bf16* __restrict__ czf, bf16* __restrict__ w,
                                                                int N, int Np) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  bf16* cl = wl + 32 * kLdw;
  float* lg = reinterpret_cast<float*>(smem + kWFixedSmem);
  const int b = blockIdx.x / Np, i = blockIdx.x % Np;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  if (i >= N) {   // padded query rows: zero weights (their outputs are dropped)
    for (int q = tid; q < NH * Np; q += kWThreads)
      w[((size_t)(b * NH + q / Np) * Np + i) * Np + q % Np] = f2bf(0.f);
    return;
  }
  stage_weights(wl, wzf, NH, 32);
  stage_bias(cl, czf, NH, 32);
  __syncthreads();

  const int rho = lane & 31, h = lane >> 5;
  const bf16* zrow = z + ((size_t)b * N + i) * N * CZ;
  const uint8_t* mrow = mask + ((size_t)b * N + i) * N;
  for (int t = wave; t < Np / 32; t += kWThreads / 64) {
    const int j0 = t * 32;
    const int jj = j0 + perm32(rho);
    const bool valid = jj < N;
    float v[64];
    bf16x8 x[8];
    load_half_row_f32(zrow + (size_t)(valid ? jj : 0) * CZ, h, valid, v);
    normalize_half_row(v, valid, x);
    // D lane (n = head, h): keys j0 + 16h + u
    const f32x16 acc = proj_block_cm_f(x, bias_step_x(valid, h), wl, cl, 0, rho, h);
    if (rho < NH) {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int j = j0 + 16 * h + u;
        lg[rho * Np + j] = j >= N ? -INFINITY : (mrow[j] ? acc[u] : -1e6f);
      }
    }
  }
  __syncthreads();
  // Softmax over j: wave w handles heads 2w, 2w + 1.
#pragma unroll 1
  for (int hd = 2 * wave; hd < 2 * wave + 2; ++hd) {
    const float* r = lg + hd * Np;
    float mx = -INFINITY;
    for (int j = lane; j < Np; j += 64) mx = fmaxf(mx, r[j]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.f;
    for (int j = lane; j < Np; j += 64) sum += fast_exp2((r[j] - mx) * kLog2e);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    const float inv = 1.0f / sum;
    bf16* wo = w + ((size_t)(b * NH + hd) * Np + i) * Np;
    for (int j = lane; j < Np; j += 64) wo[j] = f2bf(fast_exp2((r[j] - mx) * kLog2e) * inv);
  }
}

// ---------------------------------------------------------------------------
// Projections of the MSA tokens: tile = (b, MSA row s, 32 tokens).  Lane
// (rho, h) holds channels 32h .. 32h+31 of token i0 + perm32(rho); the
// LayerNorm (64 channels) is affine-free against the folded Wm | Wg (512 rows
// in LDS, stride kLdw64) plus one bias k-step.
// ---------------------------------------------------------------------------
constexpr int kPThreads = 512;
constexpr int kPRows = 2 * HC;
constexpr int kPSmem = kPRows * kLdw64 * 2 + kPRows * 2 * 2;

__device__ __forceinline__ f32x16 proj64_cm(const bf16x8 x[4], bf16x8 xb, const bf16* wl, const bf16* cl, int row0,
                                            int n, int h) {
  f32x16 acc = zero16();
  const bf16* w = wl + (row0 + n) * kLdw64 + 32 * h;
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma32(x[s], load8(w + 8 * s), acc);
  return mfma32(xb, bias_step_w(cl, row0 + n, h), acc);
}

__device__ __forceinline__ f32x16 proj64_pm(const bf16x8 x[4], bf16x8 xb, const bf16* wl, const bf16* cl, int row0,
                                            int n, int h) {
  f32x16 acc = zero16();
  const int r = row0 + perm32(n);
  const bf16* w = wl + r * kLdw64 + 32 * h;
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma32(load8(w + 8 * s), x[s], acc);
  return mfma32(bias_step_w(cl, r, h), xb, acc);
}

__global__ __launch_bounds__(kPThreads) void pwa_proj_kernel(const bf16* __restrict__ m, const bf16* __restrict__ wf,
                                                             const bf16* __restrict__ cf, bf16* __restrict__ vt,
                                                             bf16* __restrict__ g, int B, int S, int S8, int N,
                                                             int Np) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  bf16* cl = wl + kPRows * kLdw64;
  for (int q = threadIdx.x; q < kPRows * (CM / 8); q += kPThreads) {
    const int r = q / (CM / 8), part = q % (CM / 8);
    store8(wl + r * kLdw64 + part * 8, load8(wf + (size_t)r * CM + part * 8));
  }
  stage_bias(cl, cf, kPRows, kPRows);
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rho = lane & 31, h = lane >> 5;
  const int waves = kPThreads / 64;
  const unsigned tpr = Np / 32;
  const unsigned ntiles = (unsigned)B * S8 * tpr;
  // Software pipeline over this wave's tiles: tile t + stride's m half-rows
  // are loaded before tile t's stores and normalised after them (vector-
  // memory counters retire in issue order, so that wait does not wait for
  // the stores).  The loads are unconditional (row 0 for slots outside the
  // sequence, zeroed when normalised).
  const unsigned stride = gridDim.x * waves;
  bf16x8 raw[4];
  auto fetch = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tpr, S8);
    const int ii = ti.col * 32 + perm32(rho);
    const bool valid = ii < N && ti.row < S;
    const bf16* row = m + (((size_t)ti.b * S + (valid ? ti.row : 0)) * N + (valid ? ii : 0)) * CM + 32 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q) raw[q] = load8(row + 8 * q);
  };
  bf16x8 x[4], xb;
  auto prepare = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tpr, S8);
    const int ii = ti.col * 32 + perm32(rho);
    const bool valid = ii < N && ti.row < S;
    float v[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) unpack8(valid ? raw[q] : bf16x8{}, v + 8 * q);
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < 32; ++c) sum += v[c];
    sum += __shfl_xor(sum, 32);
    const float mean = sum * (1.0f / CM);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const float d = v[c] - mean;
      ss += d * d;
    }
    ss += __shfl_xor(ss, 32);
    const float rstd = valid ? rsqrtf(ss * (1.0f / CM) + 1e-5f) : 0.f;
#pragma unroll
    for (int c = 0; c < 32; ++c) x[c >> 3][c & 7] = f2bf((v[c] - mean) * rstd);
    xb = bias_step_x(valid, h);
  };

  unsigned t = blockIdx.x * waves + wave;
  if (t < ntiles) {
    fetch(t);
    prepare(t);
  }
  for (; t < ntiles; t += stride) {
    const unsigned tn = t + stride;
    if (tn < ntiles) fetch(tn);
    const TileIdx ti = split_tile(t, tpr, S8);
    const int it = ti.col, s = ti.row, b = ti.b;
    const int i0 = it * 32;
    const int ii = i0 + perm32(rho);
    // v^T: D lane (n = channel within head cb, h) holds tokens i0 + 16h + u.
    // (Both output loops are unrolled, one block per scheduling region, so
    // that the compiler sees every store when it places the wait for the
    // next tile's loads.)
#pragma unroll
    for (int cb = 0; cb < NH; ++cb) {
      const f32x16 a = proj64_cm(x, xb, wl, cl, cb * 32, rho, h);
      float r[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) r[u] = a[u];
      store16(vt + ((((size_t)b * NH + cb) * S8 + s) * CH + rho) * Np + i0 + 16 * h, r);
      __builtin_amdgcn_sched_barrier(0);
    }
    // g: D lane (n = token slot perm32(n), h) holds channels cb*32 + 16h + u.
#pragma unroll
    for (int cb = 0; cb < NH; ++cb) {
      const f32x16 a = proj64_pm(x, xb, wl, cl, HC + cb * 32, rho, h);
      float r[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) r[u] = sigmoidf_fast(a[u]);
      store16(g + (((size_t)b * S8 + s) * Np + ii) * HC + cb * 32 + 16 * h, r);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (tn < ntiles) prepare(tn);
  }
}

// ---------------------------------------------------------------------------
// Contraction fused with the gate and the output projection.
// Workgroup = (b, 8 MSA rows s0.., 128 query rows i0..); 8 waves, wave
// (wi = wave & 1, ws = wave >> 1) owns rows i0 + 64 wi .. +63 of MSA rows
// s0 + 2 ws and s0 + 2 ws + 1.  For each head h:
//   O_h[i][(s, d)] = sum_j W[b][h][i][j] V^T[b][h][(s, d)][j]    (MFMA, K = Np,
//     64-deep k-tiles copied straight into LDS, double-buffered across heads)
//   out^T[o][i] += sum_d Wo[o][h*32 + d] (g[b][s][i][h*32 + d] O_h[i][(s, d)])
// with the gated O_h taken from the accumulator registers as the B operand of
// the projection (Wo in LDS).  After the 8 heads the 64 output channels (+ m)
// are written once: neither g * o nor o ever goes to HBM.  Per 16-deep k-step
// a wave reads 4 operand fragments (W rows of its two i blocks, V^T rows of
// its two MSA rows) for 4 MFMAs.
// ---------------------------------------------------------------------------
constexpr int kFuThreads = 512;
constexpr int kFuI = 128;                       // query rows per workgroup
constexpr int kFuS = 8;                         // MSA rows per workgroup (2 per wave)
constexpr int kFuBK = 64;
constexpr int kFuWTile = kFuI * kFuBK;          // W tile: [128 rows][8 chunks of 8]
constexpr int kFuVTile = kFuS * CH * kFuBK;     // V^T tile: [256 rows (s, d)][8 chunks of 8]
constexpr int kFuStage = kFuWTile + kFuVTile;
constexpr int kLdwO = HC + 8;                   // Wo row stride in LDS
constexpr int kFuSmem = 2 * kFuStage * 2 + CM * kLdwO * 2;

__global__ __launch_bounds__(kFuThreads) void pwa_fused_kernel(const bf16* __restrict__ w,
                                                               const bf16* __restrict__ vt,
                                                               const bf16* __restrict__ g,
                                                               const bf16* __restrict__ wo, const bf16* mres,
                                                               bf16* out, int8_t* tail, int S, int S8, int N, int Np,
                                                               int residual, int nitems) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  bf16* wol = smem + 2 * kFuStage;
  // XCD-aware: consecutive items (the i-tiles of one s-tile, which read the
  // same V^T rows) land on one XCD.
  const int per_xcd = gridDim.x / kNtXcds;
  const int item = (blockIdx.x % kNtXcds) * per_xcd + blockIdx.x / kNtXcds;
  if (item >= nitems) return;   // before any barrier: the whole workgroup leaves
  const int nit = Np / kFuI, nst = S8 / kFuS;
  const int it = item % nit, st = (item / nit) % nst, b = item / (nit * nst);
  const int i0 = it * kFuI, s0 = st * kFuS;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, lh = lane >> 5;
  const int wi = wave & 1, ws = wave >> 1;

  for (int q = tid; q < CM * (HC / 8); q += kFuThreads) {
    const int r = q / (HC / 8), part = q % (HC / 8);
    store8(wol + r * kLdwO + part * 8, load8(wo + (size_t)r * HC + part * 8));
  }

  // The W tile (128 rows x 128 B) is 16 copies of 1 KB, the V^T tile (256
  // rows) 32; wave w moves W copies w, w + 8 and V^T copies w, w + 8, w + 16,
  // w + 24.  Copy j writes LDS chunk 64 j + lane of its tile.
  unsigned voff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int p = (wave + 8 * q) * 64 + lane, r = p >> 3, c = (p & 7) ^ nt_swz(p >> 3);
    voff[q] = (unsigned)(r * Np + c * 8) * 2;
  }
  auto rsrcs = [&](int h, __amdgpu_buffer_rsrc_t& rw, __amdgpu_buffer_rsrc_t& rv) {
    rw = buffer_rsrc(w + ((size_t)(b * NH + h) * Np + i0) * Np, (unsigned)kFuI * Np * 2);
    rv = buffer_rsrc(vt + (((size_t)(b * NH + h) * S8 + s0) * CH) * Np, (unsigned)(kFuS * CH) * Np * 2);
  };
  auto stage = [&](__amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rv, int kt, int buf) {
    bf16* stg = smem + buf * kFuStage;
    const unsigned soff = (unsigned)(kt * kFuBK) * 2;
#pragma unroll
    for (int q = 0; q < 2; ++q) nt_copy16_to_lds(rw, stg + (wave + 8 * q) * 512, voff[q], soff);
#pragma unroll
    for (int q = 0; q < 4; ++q) nt_copy16_to_lds(rv, stg + kFuWTile + (wave + 8 * q) * 512, voff[q], soff);
  };

  const int nk = Np / kFuBK;
  int jrow[2], offi[2];
#pragma unroll
  for (int si = 0; si < 2; ++si) jrow[si] = (2 * ws + si) * 32 + perm32(ln);
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) offi[ib] = wi * 64 + ib * 32 + ln;

  f32x16 oacc[2][2][2];   // [si][ob][ib]: out^T rows ob*32.., columns i, MSA row s0 + 2 ws + si
#pragma unroll
  for (int si = 0; si < 2; ++si)
#pragma unroll
    for (int ob = 0; ob < 2; ++ob)
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) oacc[si][ob][ib] = zero16();

  __amdgpu_buffer_rsrc_t rw, rv;
  rsrcs(0, rw, rv);
  stage(rw, rv, 0, 0);
  int gk = 0;   // running k-tile index: LDS buffer gk & 1
#pragma unroll 1
  for (int h = 0; h < NH; ++h) {
    f32x16 acc[2][2];   // [si][ib]
#pragma unroll
    for (int si = 0; si < 2; ++si)
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) acc[si][ib] = zero16();
#pragma unroll 1
    for (int kt = 0; kt < nk; ++kt, ++gk) {
      __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of the k-tile landed
      __syncthreads();                       // ... and everyone's; the other buffer is free again
      if (kt + 1 < nk) {
        stage(rw, rv, kt + 1, (gk + 1) & 1);
      } else if (h + 1 < NH) {
        rsrcs(h + 1, rw, rv);
        stage(rw, rv, 0, (gk + 1) & 1);
      }
      const bf16* sa = smem + (gk & 1) * kFuStage;
      const bf16* sb = sa + kFuWTile;
      // fragments of k-step ks + 1 are read while k-step ks is multiplied
      bf16x8 fj[2][2], fi[2][2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        fj[0][x] = load8(sb + nt_off(jrow[x], lh));
        fi[0][x] = load8(sa + nt_off(offi[x], lh));
      }
#pragma unroll
      for (int ks = 0; ks < kFuBK / 16; ++ks) {
        const int c = ks & 1;
        if (ks + 1 < kFuBK / 16) {
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            fj[c ^ 1][x] = load8(sb + nt_off(jrow[x], 2 * (ks + 1) + lh));
            fi[c ^ 1][x] = load8(sa + nt_off(offi[x], 2 * (ks + 1) + lh));
          }
        }
#pragma unroll
        for (int si = 0; si < 2; ++si)
#pragma unroll
          for (int ib = 0; ib < 2; ++ib) acc[si][ib] = mfma32(fj[c][si], fi[c][ib], acc[si][ib]);
      }
    }
    // acc[si][ib] lane (ln, lh) register u <-> O_h[i = i0 + wi*64 + ib*32 + ln][(s0 + 2 ws + si, d = 16 lh + u)]
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      const int s = s0 + 2 * ws + si;
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const int i = i0 + offi[ib];
        const bf16* gp = g + (((size_t)b * S8 + s) * Np + i) * HC + h * CH + 16 * lh;
        const bf16x8 g0 = load8(gp), g1 = load8(gp + 8);
        bf16x8 go0, go1;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          go0[u] = f2bf(acc[si][ib][u] * bf2f(g0[u]));
          go1[u] = f2bf(acc[si][ib][8 + u] * bf2f(g1[u]));
        }
#pragma unroll
        for (int ob = 0; ob < 2; ++ob) {
          const bf16* wrow = wol + (ob * 32 + perm32(ln)) * kLdwO + h * CH + 16 * lh;
          oacc[si][ob][ib] = mfma32(load8(wrow), go0, oacc[si][ob][ib]);
          oacc[si][ob][ib] = mfma32(load8(wrow + 8), go1, oacc[si][ob][ib]);
        }
      }
    }
  }
  // oacc[si][ob][ib] lane (ln, lh) register u <-> out channel ob*32 + 16 lh + u of (s, i0 + offi[ib])
#pragma unroll
  for (int si = 0; si < 2; ++si) {
    const int s = s0 + 2 * ws + si;
    if (s >= S) continue;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int i = i0 + offi[ib];
      if (i >= N) continue;
#pragma unroll
      for (int ob = 0; ob < 2; ++ob) {
        const size_t off = (((size_t)b * S + s) * N + i) * CM + ob * 32 + 16 * lh;
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = oacc[si][ob][ib][u];
        if (residual && tail) {   // residual stream with an int8 tail (common.h), in place
          float mv[16];
          tail_decode16(load8(mres + off), load8(mres + off + 8), load_tail16(tail + off), mv);
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] += mv[u];
          tail_store16(out + off, tail + off, v);
          continue;
        }
        if (residual) {
          const bf16x8 r0 = load8(mres + off), r1 = load8(mres + off + 8);
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
}

struct PwaLayout {
  int64_t Np, S8;
  size_t w, vt, g, wzf, czf, wmf, cmf, total;
};

PwaLayout pwa_layout(int64_t B, int64_t S, int64_t N) {
  PwaLayout L;
  L.Np = round_up(N, kNtTile);
  L.S8 = round_up(S, 8);
  size_t p = 0;
  L.w = p;
  p += round_up((size_t)B * NH * L.Np * L.Np * 2, 256);
  L.vt = p;
  p += round_up((size_t)B * NH * L.S8 * CH * L.Np * 2, 256);
  L.g = p;
  p += round_up((size_t)B * L.S8 * L.Np * HC * 2, 256);
  L.wzf = p;
  L.czf = p + round_up((size_t)NH * CZ * 2, 256);
  p += fold_bytes(NH);
  L.wmf = p;
  L.cmf = p + round_up((size_t)kPRows * CM * 2, 256);
  p += fold_bytes(kPRows, CM);
  L.total = p;
  return L;
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_pwa_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_m, int64_t c_h, int64_t H) {
  if (B <= 0 || S <= 0 || N <= 0 || c_m != CM || c_h != CH || H != NH) return 0;
  return pwa_layout(B, S, N).total;
}

extern "C" int bioemu_pwa_fwd(const void* m, const void* z, const uint8_t* mask, const float* norm_m_w,
                              const float* norm_m_b, const void* w_m, const void* w_g, const float* norm_z_w,
                              const float* norm_z_b, const void* w_z, const void* w_o, void* out, int8_t* res_tail,
                              void* workspace, size_t workspace_bytes, int64_t B, int64_t S, int64_t N, int64_t c_m,
                              int64_t c_z, int64_t c_h, int64_t H, int residual, hipStream_t stream) {
  if (c_m != CM || c_z != CZ || c_h != CH || H != NH)
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "pwa: only c_m=64, c_z=128, c_h=32, 8 heads are supported (got %lld, %lld, %lld, %lld)",
                     (long long)c_m, (long long)c_z, (long long)c_h, (long long)H);
  if (B <= 0 || S <= 0 || N <= 0 || B > 65535 || N > 4096 || S > 65535)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: bad shape B=%lld S=%lld N=%lld", (long long)B, (long long)S,
                     (long long)N);
  if (!m || !z || !mask || !norm_m_w || !norm_m_b || !w_m || !w_g || !norm_z_w || !w_z || !w_o || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: null pointer argument");
  if (!aligned16(m) || !aligned16(z) || !aligned16(out) || !aligned16(w_m) || !aligned16(w_g) || !aligned16(w_z) ||
      !aligned16(w_o) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: tensors and workspace must be 16-byte aligned");
  if (out == m && !residual) return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: out may alias m only with residual=1");
  if (res_tail && (!residual || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: res_tail needs residual=1 and 16-byte alignment");
  const PwaLayout L = pwa_layout(B, S, N);
  if (workspace_bytes < L.total)
    return set_error(BIOEMU_ERR_WORKSPACE, "pwa: workspace %zu < required %zu", workspace_bytes, L.total);
  if ((int64_t)kNtTile * L.Np * 2 > 0xffffffffLL || (int64_t)L.S8 * CH > (1 << 24))
    return set_error(BIOEMU_ERR_UNSUPPORTED, "pwa: shape too large");
  char* ws = static_cast<char*>(workspace);
  bf16* wbuf = reinterpret_cast<bf16*>(ws + L.w);
  bf16* vt = reinterpret_cast<bf16*>(ws + L.vt);
  bf16* gbuf = reinterpret_cast<bf16*>(ws + L.g);
  bf16* wzf = reinterpret_cast<bf16*>(ws + L.wzf);
  bf16* czf = reinterpret_cast<bf16*>(ws + L.czf);
  bf16* wmf = reinterpret_cast<bf16*>(ws + L.wmf);
  bf16* cmf = reinterpret_cast<bf16*>(ws + L.cmf);

  if (B * L.S8 * (L.Np / 32) >= kMaxTiles) return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: too many row tiles");
  int rc = launch_fold_ln(w_z, norm_z_w, norm_z_b, wzf, czf, NH, stream);
  if (!rc) rc = launch_fold_ln2(w_m, w_g, HC, norm_m_w, norm_m_b, wmf, cmf, 2 * HC, stream, CM);
  if (rc) return rc;

  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const int Np = (int)L.Np, S8 = (int)L.S8;

  const size_t wsmem = kWFixedSmem + (size_t)NH * Np * 4;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(pwa_weights_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)wsmem) != hipSuccess ||
      hipFuncSetAttribute(reinterpret_cast<const void*>(pwa_proj_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          kPSmem) != hipSuccess ||
      hipFuncSetAttribute(reinterpret_cast<const void*>(pwa_fused_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kFuSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "pwa: cannot set dynamic LDS size");
  {
    KernelTimerScope timed("pwa_weights", stream);
    hipLaunchKernelGGL(pwa_weights_kernel, dim3((unsigned)(B * Np)), dim3(kWThreads), wsmem, stream,
                       static_cast<const bf16*>(z), mask, wzf, czf, wbuf, (int)N, Np);
  }
  rc = check_launch("pwa_weights");
  if (rc) return rc;
  {
    const long long tiles = B * S8 * (Np / 32);
    const unsigned grid = (unsigned)std::min<long long>(2LL * cus, (tiles + 7) / 8);
    KernelTimerScope timed("pwa_proj", stream);
    hipLaunchKernelGGL(pwa_proj_kernel, dim3(grid), dim3(kPThreads), kPSmem, stream, static_cast<const bf16*>(m),
                       wmf, cmf, vt, gbuf, (int)B, (int)S, S8, (int)N, Np);
  }
  rc = check_launch("pwa_proj");
  if (rc) return rc;
  {
    const long long items = B * (S8 / kFuS) * (Np / kFuI);
    const long long grid = (items + kNtXcds - 1) / kNtXcds * kNtXcds;
    if (grid > 0x7fffffffLL) return set_error(BIOEMU_ERR_INVALID_ARG, "pwa: too many work items");
    KernelTimerScope timed("pwa_fused", stream);
    hipLaunchKernelGGL(pwa_fused_kernel, dim3((unsigned)grid), dim3(kFuThreads), kFuSmem, stream, wbuf, vt, gbuf,
                       static_cast<const bf16*>(w_o), static_cast<const bf16*>(m), static_cast<bf16*>(out), res_tail,
                       (int)S, S8, (int)N, Np, residual, (int)items);
  }
  return check_launch("pwa_fused");
}
