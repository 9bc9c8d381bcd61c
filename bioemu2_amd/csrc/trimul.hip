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
// Padded planes (Np = N rounded up to the 256 contraction tile) are zero in every padded row and
// column, so the contraction needs no edge handling and padding never changes
// a valid output bit.
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int D = 128;               // pair channels (c_z)

// ---------------------------------------------------------------------------
// Stage 1: LN_in + gated input projection + mask, channel-major output.
//
// Tile = (b, frame row i, 32 frame columns); frame (i, k) is x[i][k]
// (outgoing) or x[k][i] (incoming).  The LayerNorm'd tile stays in registers
// as MFMA operands (pairtile.h); p_in and g_in (512 x 128) sit in LDS for the
// whole persistent workgroup.  A masked pair's LayerNorm row is zeroed before
// the bias-free projections, so its p is exactly 0 and so is p * sigmoid(g):
// the masked_fill of the reference (triangle_multiplication.py:93).  Rows and
// columns in [N, Np) come out zero, which the padded contraction relies on.
// Output: a and b as channel-major planes [B][D][Np][Np] (k contiguous).
// ---------------------------------------------------------------------------
// Workgroup size: kWaves = 8 or 12 waves, chosen per launch (in_waves_per_wg);
// the staged weights (140 KB of LDS) allow one workgroup per CU, so kWaves
// waves share 4 SIMDs and the launch bound 64 * kWaves gives each wave the
// register budget of its occupancy (256 VGPRs at 8 waves, 168 at 12).
constexpr int kInRows = 4 * D;                 // p_in (2D rows) then g_in (2D rows)
constexpr int kInSmem = kInRows * kLdw * 2 + 2 * D * 4;   // weights, then LayerNorm gamma | beta (fp32)

// Waves per workgroup (pick_waves_per_wg).  Measured with whole rounds of
// tiles: 12 waves give 1.02x the throughput of 8 at N = 768.  (16 waves would
// cap a wave at 128 VGPRs, which spills.)  Picks: N = 512 -> 8, 768 -> 12.
inline int in_waves_per_wg(long long tiles, int cus) {
  static const int waves[2] = {8, 12};
  static const double gain[2] = {1.0, 1.02};
  return pick_waves_per_wg(tiles, cus, waves, gain, 2);
}

template <bool kOutgoing, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void trimul_proj_in_kernel(
    const bf16* __restrict__ x, const uint8_t* __restrict__ mask, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ p_w, const bf16* __restrict__ g_w,
    bf16* __restrict__ ab, int B, int N, int Np) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  // gamma and beta live in LDS: read from global memory inside the tile loop
  // they would be vector-memory loads issued after the previous tile's
  // stores, and waiting for them would wait for those stores.
  float* lnl = reinterpret_cast<float*>(smem + kInRows * kLdw * 2);
  stage_weights(wl, p_w, 2 * D, 2 * D);
  stage_weights(wl + 2 * D * kLdw, g_w, 2 * D, 2 * D);
  for (int q = threadIdx.x; q < D; q += blockDim.x) {
    lnl[q] = ln_w[q];
    lnl[D + q] = ln_b[q];
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rho = lane & 31, h = lane >> 5;
  constexpr int waves = kWaves;
  const unsigned tiles_per_row = Np / 32;
  const unsigned ntiles = (unsigned)B * Np * tiles_per_row;
  const size_t plane = (size_t)Np * Np;

  // Software pipeline over this wave's tiles: tile t + stride's inputs (this
  // lane's half of its pair's x row and the pair's mask byte) are loaded
  // before tile t's stores are issued and normalised after them.  Vector-
  // memory counters retire in issue order, so waiting for those loads then
  // does not wait for the stores to be written.  The loads are unconditional
  // (pair 0 for slots outside the sequence; such slots are zeroed through
  // `keep`) so that nothing touches their destination registers, or reads the
  // mask byte, before the wait.
  const unsigned stride = gridDim.x * waves;
  bf16x8 raw[8];
  uint8_t mraw = 0;
  bool inb_next = false;
  auto fetch = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tiles_per_row, Np);
    const int i = ti.row, b = ti.b, kk = ti.col * 32 + perm32(rho);
    inb_next = i < N && kk < N;
    const size_t pair = !inb_next ? 0 : kOutgoing ? ((size_t)b * N + i) * N + kk : ((size_t)b * N + kk) * N + i;
    mraw = mask[pair];
    const bf16* row = x + pair * D + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) raw[s] = load8(row + 16 * s);
  };
  bf16x8 xf[8];
  auto prepare = [&]() {
    layernorm_half_row(raw, lnl, lnl + D, h, 1e-5f, xf);
    if (!(inb_next && mraw != 0)) {
#pragma unroll
      for (int s = 0; s < 8; ++s) xf[s] = bf16x8{};
    }
  };

  unsigned t = blockIdx.x * waves + wave;
  if (t < ntiles) {
    fetch(t);
    prepare();
  }
  for (; t < ntiles; t += stride) {
    const unsigned tn = t + stride;
    if (tn < ntiles) fetch(tn);
    const TileIdx ti = split_tile(t, tiles_per_row, Np);
    const int kt = ti.col, i = ti.row, b = ti.b;
    const int k0 = kt * 32;
#pragma unroll 1
    for (int blk = 0; blk < 8; ++blk) {   // a: blk 0..3, b: blk 4..7 (32 channels each)
      const f32x16 pa = proj_block_cm(xf, wl, blk * 32, rho, h);
      const f32x16 ga = proj_block_cm(xf, wl, 2 * D + blk * 32, rho, h);
      // Lane (rho, h) holds columns 16h .. 16h + 15 of channel ch as two
      // 8-column chunks.  Lanes rho and rho ^ 16 swap their second chunks, so
      // that each of the two stores writes whole 64-byte column runs: the
      // first those of channels with rho < 16 (4 lanes each), the second
      // those of the other 16 channels.
      bf16x8 first, second, recv;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        first[u] = f2bf(pa[u] * sigmoidf_fast(ga[u]));
        second[u] = f2bf(pa[8 + u] * sigmoidf_fast(ga[8 + u]));
      }
      {
        const u32x4 sw = __builtin_bit_cast(u32x4, second);
        u32x4 rw;
#pragma unroll
        for (int d = 0; d < 4; ++d) rw[d] = (unsigned)__shfl_xor((int)sw[d], 16);
        recv = __builtin_bit_cast(bf16x8, rw);
      }
      const int which = blk >> 2, ch = (blk & 3) * 32 + rho;
      bf16* own = ab + ((size_t)(which * B + b) * D + ch) * plane + (size_t)i * Np + k0 + 16 * h;
      bf16* partner = own + (rho < 16 ? 16 : -16) * (long long)plane + 8;   // channel ch ^ 16, columns + 8
      const bool low = rho < 16;   // per-lane selects: two store instructions for the whole wave
      store8(low ? own : partner, low ? first : recv);
      store8(low ? partner : own, low ? recv : first);
    }
    if (tn < ntiles) prepare();
  }
}

// ---------------------------------------------------------------------------
// Stage 3 prep: fold the two LayerNorm affines into the output projections.
//   p_out(LN_out(o)) = xhat_o (Wp diag(g_out))^T + Wp b_out
//   g_out(LN_in(x))  = xhat_x (Wg diag(g_in))^T  + Wg b_in
// with xhat the normalised (affine-free) rows.  One workgroup per output row.
// fold layout: [Wp' (D x D) | Wg' (D x D)] bf16, then [cp (D) | cg (D)] fp32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(D) void trimul_fold_kernel(const bf16* __restrict__ p_w, const bf16* __restrict__ g_w,
                                                      const float* __restrict__ ln_out_w,
                                                      const float* __restrict__ ln_out_b,
                                                      const float* __restrict__ ln_in_w,
                                                      const float* __restrict__ ln_in_b, bf16* __restrict__ wfold,
                                                      float* __restrict__ cfold) {
  __shared__ float red[2][D];
  const int e = blockIdx.x, c = threadIdx.x;
  const float wp = bf2f(p_w[e * D + c]), wg = bf2f(g_w[e * D + c]);
  wfold[e * D + c] = f2bf(wp * ln_out_w[c]);
  wfold[D * D + e * D + c] = f2bf(wg * ln_in_w[c]);
  red[0][c] = wp * ln_out_b[c];
  red[1][c] = wg * ln_in_b[c];
  __syncthreads();
  for (int st = D / 2; st > 0; st >>= 1) {
    if (c < st) {
      red[0][c] += red[0][c + st];
      red[1][c] += red[1][c + st];
    }
    __syncthreads();
  }
  if (c == 0) {
    cfold[e] = red[0][0];
    cfold[D + e] = red[1][0];
  }
}

// Affine-free LayerNorm of the 128 channels held by lanes l and l^32, bf16
// result in the MFMA operand layout (pairtile.h); v holds this lane's 64.
__device__ __forceinline__ void normalize_half_row(const float* v, bf16x8 out[8]) {
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < 64; ++c) sum += v[c];
  sum += __shfl_xor(sum, 32);
  const float mean = sum * (1.0f / D);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < 64; ++c) {
    const float d = v[c] - mean;
    ss += d * d;
  }
  ss += __shfl_xor(ss, 32);
  const float rstd = rsqrtf(ss * (1.0f / D) + 1e-5f);
#pragma unroll
  for (int c = 0; c < 64; ++c) out[c >> 3][c & 7] = f2bf((v[c] - mean) * rstd);
}

// ---------------------------------------------------------------------------
// Stage 3: out = p_out(LN_out(o)) * sigmoid(g_out(LN_in(x)))  (+ x).
//
// Tile = (b, row i, 32 columns j), one per wave at a time.  o is channel-major
// (the contraction's output planes): a tile's o block, 128 channels x one
// 64-byte run, is read with 16-byte loads and turned pair-major through a
// per-wave LDS buffer; x is pair-major.  Both LayerNorms run affine-free in
// registers against the folded weights, which sit in LDS with the folded
// biases.
//
// Channel interleave (pairtile.h): the two lanes (rho, 0) and (rho, 1) of a
// pair hold alternate 8-channel chunks, lane h chunk s = channels
// 16 s + 8 h + (0..7), which is the MFMA B operand of k-step s.  The output
// stores use the same interleave.  Output lanes: LDS row 32 cb + m of each folded
// weight half holds weight row 32 cb + 16 ((m & 15) >> 3) + 8 (m >> 4) +
// (m & 7), so that lane (rho, h) of output block cb holds channels
// 32 cb + 8 h + u and 32 cb + 16 + 8 h + u (u < 8): x chunks 2 cb and
// 2 cb + 1 of its own registers, which supply the residual.  Tail bytes
// (16 per load or store, contiguous channels 32 cb + 16 h + 0..15) are
// exchanged between the two lanes of a pair.
//
// Software pipeline: tile t + stride's x and o loads are issued before tile
// t's stores and consumed after them; vector-memory counters retire in issue
// order, so waiting for the loads does not wait for the stores.
// ---------------------------------------------------------------------------
constexpr int kOutThreads = 512;
constexpr int kOutWaves = kOutThreads / 64;
constexpr int kOutPlaneSpan = 23;       // planes past its base that one o copy instruction reaches
constexpr int kOutTile = D * 32 + 32;   // per-wave o buffer, bf16 elements
constexpr int kOutSmem = 2 * D * kLdw * 2 + 2 * D * 4 + kOutWaves * kOutTile * 2;

// Element offset of (channel c, column j) in a wave's o buffer: 64-byte
// channel rows in eight 1 KB blocks, block q holding channels
// 32 (q & 3) + 8 (q >> 2) + {0..7, 16..23}, and blocks 4..7 (channel bit 3
// set) 64 bytes further on, so that the two half-waves' reads (channels c and
// c + 8 of the same 32 columns) use different LDS banks; each block is what
// one 16-byte copy instruction writes.
__device__ __forceinline__ int obuf_off(int c, int j) {
  const int q = 4 * ((c >> 3) & 1) + (c >> 5), slot = 8 * ((c >> 4) & 1) + (c & 7);
  return q * 512 + slot * 32 + j + ((q >> 2) << 5);
}

// Lanes of pair slots past N store into `discard` (a dead workspace region,
// 16 KB) instead of skipping the store: a conditional store would hide the
// number of stores from the compiler's wait counting, which would then wait
// for the stores before the next tile's data.
// With kTail the residual stream also has an int8 tail plane (common.h):
// x + tail is read, and the sum is written back as out + tail (in place).
template <bool kTail>
__global__ __launch_bounds__(kOutThreads) void trimul_out_kernel(
    const bf16* __restrict__ o, const bf16* x, const bf16* __restrict__ wfold, const float* __restrict__ cfold,
    bf16* out, int8_t* tail, bf16* __restrict__ discard, int B, int N, int Np, int residual) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  float* cl = reinterpret_cast<float*>(smem + 2 * D * kLdw * 2);
  bf16* obuf = reinterpret_cast<bf16*>(smem + 2 * D * kLdw * 2 + 2 * D * 4);
  for (int q = threadIdx.x; q < 2 * D * (D / 8); q += blockDim.x) {
    const int r = q >> 4, part = q & 15;
    const int half = r / D, cb = (r % D) >> 5, m = r & 31;
    const int src = half * D + 32 * cb + 16 * ((m & 15) >> 3) + 8 * (m >> 4) + (m & 7);
    store8(wl + r * kLdw + part * 8, load8(wfold + (size_t)src * D + part * 8));
  }
  // cl[half D + 64 h + 16 cb + u]: bias of the channel lane h holds in register u of block cb
  for (int t = threadIdx.x; t < 2 * D; t += blockDim.x) {
    const int e = t % D, h = e >> 6, cb = (e >> 4) & 3, u = e & 15;
    cl[t] = cfold[t - e + 32 * cb + 16 * (u >> 3) + 8 * h + (u & 7)];
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rho = lane & 31, h = lane >> 5;
  const unsigned tiles_per_row = (N + 31) / 32;
  const unsigned ntiles = (unsigned)B * N * tiles_per_row;
  const unsigned stride = gridDim.x * kOutWaves;
  const size_t plane = (size_t)Np * Np;
  bf16* ob = obuf + wave * kOutTile;

  // Next tile's raw inputs.  o channel 32 (q & 3) + 8 (q >> 2) + 16 (s >> 3) +
  // (s & 7), s = lane >> 2, columns j0 + 8 (lane & 3) .. + 7 go straight from
  // global memory into the wave's o buffer (buffer loads that write LDS: no
  // registers; instruction q writes block q, 1 KB contiguously); this lane's
  // x chunks (and the tail bytes) go to registers.  Columns of the
  // last tile of a row may reach past N but stay below Np (o is Np wide).
  // The o copies are issued first, so the wait for them in prepare() counts
  // the x / tail loads and the current tile's stores issued after them.
  bf16x8 xraw[8];
  u32x4 traw[4];
  // Copy instruction q reads channels c_q + 16 (slot >> 3) + (slot & 7),
  // c_q = 32 (q & 3) + 8 (q >> 2), through a buffer resource based at its own
  // first plane: 24 planes from that base, so 32-bit offsets hold for
  // 23 Np^2 + 32 elements (N <= 9472), the whole 128-plane span need not.
  const unsigned o_extent = (unsigned)((kOutPlaneSpan * plane + 32) * 2);
  auto fetch = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tiles_per_row, N);
    const int i = ti.row, b = ti.b, j0 = ti.col * 32;
    const bf16* obase = o + (size_t)b * D * plane + (size_t)i * Np + j0;
    const int slot = lane >> 2;
    const unsigned ovoff = ((unsigned)(16 * (slot >> 3) + (slot & 7)) * (unsigned)plane + 8u * (lane & 3)) * 2u;
#pragma unroll
    for (int q = 0; q < 8; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          buffer_rsrc(obase + (size_t)(32 * (q & 3) + 8 * (q >> 2)) * plane, o_extent),
          (__attribute__((address_space(3))) void*)(ob + 512 * q + (q >= 4 ? 32 : 0)), 16, ovoff, 0u, 0, 0);
    // Nothing may be scheduled above the copies: the wait in prepare() counts
    // every vector-memory operation issued after them.
    __builtin_amdgcn_sched_barrier(0);
    const int jj = j0 + perm32(rho);
    const size_t pair = ((size_t)b * N + i) * N + (jj < N ? jj : 0);
    const bf16* xr = x + pair * D + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) xraw[s] = load8(xr + 16 * s);
    if (kTail) {
#pragma unroll
      for (int q = 0; q < 4; ++q) traw[q] = load_tail16(tail + pair * D + 32 * q + 16 * h);
    }
  };
  // Vector-memory operations issued after a tile's o copies and before its
  // prepare(): the x (and tail) loads, then (except for a wave's first tile)
  // the previous tile's stores: two bf16 chunks, plus a tail chunk with kTail,
  // per output block.
  constexpr int kAfterLoads = 8 + (kTail ? 4 : 0);
  constexpr int kAfterOCopies = kAfterLoads + 4 * (kTail ? 3 : 2);
  // Current tile's operands: normalised o and x rows, the raw x chunks and their tails.
  bf16x8 of[8], xf[8], xres[8];
  u32x4 tres[4];
  auto prepare = [&](bool first) {
    // vmcnt <= (loads and stores issued after the o copies): this wave's o copies have landed
    if (first)
      __builtin_amdgcn_s_waitcnt(0x0f70 | (kAfterLoads & 15) | ((kAfterLoads >> 4) << 14));
    else
      __builtin_amdgcn_s_waitcnt(0x0f70 | (kAfterOCopies & 15) | ((kAfterOCopies >> 4) << 14));
    __builtin_amdgcn_sched_barrier(0);   // the o reads stay below the wait
    float v[64];
    const int p = perm32(rho);
#pragma unroll
    for (int c = 0; c < 64; ++c) v[c] = bf2f(ob[obuf_off(16 * (c >> 3) + 8 * h + (c & 7), p)]);
    normalize_half_row(v, of);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      unpack8(xraw[s], v + 8 * s);
      xres[s] = xraw[s];
    }
    if (kTail) {
#pragma unroll
      for (int q = 0; q < 4; ++q) tres[q] = exchange_tail_halves(traw[q], h);
    }
    normalize_half_row(v, xf);
  };

  unsigned t = blockIdx.x * kOutWaves + wave;
  if (t < ntiles) {
    fetch(t);
    prepare(true);
  }
  for (; t < ntiles; t += stride) {
    const unsigned tn = t + stride;
    if (tn < ntiles) fetch(tn);
    const TileIdx ti = split_tile(t, tiles_per_row, N);
    const int jj = ti.col * 32 + perm32(rho);
    const bool valid = jj < N;
    const size_t pair = ((size_t)ti.b * N + ti.row) * N + (valid ? jj : 0);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const f32x16 pa = proj_block_pm(of, wl, cb * 32, rho, h);
      const f32x16 ga = proj_block_pm(xf, wl, D + cb * 32, rho, h);
      const int e0 = 64 * h + 16 * cb;
      float r[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) r[u] = (pa[u] + cl[e0 + u]) * sigmoidf_fast(ga[u] + cl[D + e0 + u]);
      if (kTail) {
        float xv[16];
        tail_decode16(xres[2 * cb], xres[2 * cb + 1], tres[cb], xv);
#pragma unroll
        for (int u = 0; u < 16; ++u) r[u] += xv[u];
        int8_t* tdiscard = reinterpret_cast<int8_t*>(discard + 64 * D);
        bf16x8 lo, hi;
        u32x4 tb;
        tail_encode16(r, lo, hi, tb);
        bf16* dst = valid ? out + pair * D : discard + lane * D;
        store8(dst + 32 * cb + 8 * h, lo);
        store8(dst + 32 * cb + 16 + 8 * h, hi);
        int8_t* tdst = valid ? tail + pair * D : tdiscard + lane * D;
        *reinterpret_cast<u32x4*>(tdst + 32 * cb + 16 * h) = exchange_tail_halves(tb, h);
        continue;
      }
      if (residual) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          r[u] += bf2f(xres[2 * cb][u]);
          r[8 + u] += bf2f(xres[2 * cb + 1][u]);
        }
      }
      bf16x8 lo, hi;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        lo[u] = f2bf(r[u]);
        hi[u] = f2bf(r[8 + u]);
      }
      bf16* dst = valid ? out + pair * D : discard + lane * D;
      store8(dst + 32 * cb + 8 * h, lo);
      store8(dst + 32 * cb + 16 + 8 * h, hi);
    }
    if (tn < ntiles) prepare(false);
  }
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

// Launches trimul_proj_in_kernel<outgoing, waves> (waves 8 or 12).
static int launch_proj_in(bool outgoing, int waves, unsigned grid, const bf16* x, const uint8_t* mask,
                          const float* ln_w, const float* ln_b, const bf16* p_w, const bf16* g_w, bf16* ab,
                          int64_t B, int64_t N, int64_t Np, hipStream_t stream) {
  const void* k = nullptr;
  if (waves == 8)
    k = outgoing ? reinterpret_cast<const void*>(trimul_proj_in_kernel<true, 8>)
                 : reinterpret_cast<const void*>(trimul_proj_in_kernel<false, 8>);
  else if (waves == 12)
    k = outgoing ? reinterpret_cast<const void*>(trimul_proj_in_kernel<true, 12>)
                 : reinterpret_cast<const void*>(trimul_proj_in_kernel<false, 12>);
  else
    return set_error(BIOEMU_ERR_LAUNCH, "trimul_proj_in: no variant with %d waves", waves);
  if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kInSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "trimul: cannot set dynamic LDS size");
  KernelTimerScope timed("trimul_proj_in", stream);
  void* args[] = {(void*)&x, (void*)&mask, (void*)&ln_w, (void*)&ln_b, (void*)&p_w, (void*)&g_w, (void*)&ab,
                  nullptr, nullptr, nullptr};
  int b32 = (int)B, n32 = (int)N, np32 = (int)Np;
  args[7] = &b32;
  args[8] = &n32;
  args[9] = &np32;
  if (hipLaunchKernel(k, dim3(grid), dim3(64 * waves), args, kInSmem, stream) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "trimul_proj_in: launch failed");
  return 0;
}

extern "C" size_t bioemu_trimul_workspace_bytes(int64_t B, int64_t N, int64_t Dc) {
  if (B <= 0 || N <= 0 || Dc <= 0) return 0;
  const int64_t Np = round_up(N, kGemmTile);
  // a, b, o planes + the folded output weights and biases
  return (size_t)(3 * B * Dc * Np * Np) * sizeof(bf16) + (size_t)(2 * Dc * Dc) * sizeof(bf16) +
         (size_t)(2 * Dc) * sizeof(float);
}

extern "C" int bioemu_trimul_fwd(const void* x, const uint8_t* mask, const float* norm_in_w,
                                 const float* norm_in_b, const void* p_in_w, const void* g_in_w,
                                 const float* norm_out_w, const float* norm_out_b,
                                 const void* p_out_w, const void* g_out_w, void* out, int8_t* res_tail,
                                 void* workspace, size_t workspace_bytes, int64_t B, int64_t N,
                                 int64_t Dc, int outgoing, int residual, hipStream_t stream) {
  if (Dc != D) return set_error(BIOEMU_ERR_UNSUPPORTED, "trimul: channel dim %lld unsupported (must be 128)", (long long)Dc);
  if (res_tail && (!residual || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: res_tail needs residual=1 and 16-byte alignment");
  if (B <= 0 || N <= 0 || B > 65535 || N > 16384)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: bad shape B=%lld N=%lld", (long long)B, (long long)N);
  if (!x || !mask || !norm_in_w || !norm_in_b || !p_in_w || !g_in_w || !norm_out_w || !norm_out_b ||
      !p_out_w || !g_out_w || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: null pointer argument");
  // trimul_out reads a tile's contraction planes through buffer resources that
  // span 23 planes plus a row each: byte extents and offsets are 32-bit, which
  // holds for N up to 9472 (padded plane 9472^2).
  if (((uint64_t)kOutPlaneSpan * round_up(N, kGemmTile) * round_up(N, kGemmTile) + 32) * 2 > 0xffffffffull)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "trimul: N=%lld too large (N <= 9472)", (long long)N);
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
  bf16* wfold = ob + plane_elems;                                  // [2][D][D]
  float* cfold = reinterpret_cast<float*>(wfold + 2 * D * D);      // [2][D]

  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const void* kout = res_tail ? reinterpret_cast<const void*>(trimul_out_kernel<true>)
                              : reinterpret_cast<const void*>(trimul_out_kernel<false>);
  if (hipFuncSetAttribute(kout, hipFuncAttributeMaxDynamicSharedMemorySize, kOutSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "trimul: cannot set dynamic LDS size");
  const long long waves_in = (long long)B * Np * (Np / 32);
  if (waves_in >= kMaxTiles) return set_error(BIOEMU_ERR_INVALID_ARG, "trimul: too many pair tiles");
  const int in_waves = in_waves_per_wg(waves_in, cus);
  const unsigned grid1 = (unsigned)std::min<long long>(cus, (waves_in + in_waves - 1) / in_waves);
  int rc = launch_proj_in(outgoing != 0, in_waves, grid1, static_cast<const bf16*>(x), mask, norm_in_w, norm_in_b,
                          static_cast<const bf16*>(p_in_w), static_cast<const bf16*>(g_in_w), ab, B, N, Np, stream);
  if (rc) return rc;
  rc = check_launch("trimul_proj_in");
  if (rc) return rc;
  rc = launch_bgemm_nt(ab, ab + plane_elems, ob, B * D, Np, stream);
  if (rc) return rc;
  {
    KernelTimerScope timed("trimul_fold", stream);
    hipLaunchKernelGGL(trimul_fold_kernel, dim3(D), dim3(D), 0, stream, static_cast<const bf16*>(p_out_w),
                       static_cast<const bf16*>(g_out_w), norm_out_w, norm_out_b, norm_in_w, norm_in_b, wfold, cfold);
  }
  rc = check_launch("trimul_fold");
  if (rc) return rc;

  const long long waves_out = (long long)B * N * ((N + 31) / 32);
  const unsigned grid3 = (unsigned)std::min<long long>(cus, (waves_out + kOutWaves - 1) / kOutWaves);
  KernelTimerScope timed("trimul_out", stream);
  // The a/b planes are dead once the contraction has run: their first 24 KB
  // take the discarded stores (bf16 values, then tail bytes) of pair slots
  // past N.
  if (res_tail)
    hipLaunchKernelGGL(trimul_out_kernel<true>, dim3(grid3), dim3(kOutThreads), kOutSmem, stream, ob,
                       static_cast<const bf16*>(x), wfold, cfold, static_cast<bf16*>(out), res_tail, ab, (int)B,
                       (int)N, (int)Np, residual);
  else
    hipLaunchKernelGGL(trimul_out_kernel<false>, dim3(grid3), dim3(kOutThreads), kOutSmem, stream, ob,
                       static_cast<const bf16*>(x), wfold, cfold, static_cast<bf16*>(out), nullptr, ab, (int)B,
                       (int)N, (int)Np, residual);
  return check_launch("trimul_out");
}
