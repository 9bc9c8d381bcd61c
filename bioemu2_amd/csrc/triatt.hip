// Triangle attention around the starting / ending node for gfx950.
//
// The reference has no triangle attention (src/bioemu2/biomoa/modules/
// pairmixer.py:459-462 removes it).  This is AlphaFold3 supplement Alg. 14/15
// with LinearNoBias projections and the reference's attention masking
// convention: masked keys are *replaced* by -1e6 before the softmax
// (AttentionPairBias.forward, src/bioemu2/biomoa/ops/attention_pair_bias.py:184-190).
//
// Frame: the starting node works on z itself, the ending node on z^T; frame
// pair (i, j) is z[i][j] (starting) or z[j][i] (ending).  Per batch b, frame
// row i, head h:
//   zn = LN(z);  q,k,v = zn Wq^T, zn Wk^T, zn Wv^T;  g = sigmoid(zn Wg^T);
//   bias[h, j, k] = (zn Wb^T)[frame (j, k), h]
//   o[i, j] = sum_k softmax_k(q[i,j].k[i,k] / sqrt(d) + bias[h,j,k], key mask[i,k]) v[i,k]
//   update[i, j] = (g[i,j] * o[i,j]) Wo^T      (written back in z's frame)
//
// Two kernels:
//   triatt_proj  : LN + the key-side projections (k, v, bias) on MFMA with
//                  weights staged once per workgroup in LDS; writes the frame-
//                  ordered keys and values of every frame row, the bias and a
//                  frame-ordered mask.
//   triatt_flash : per (b, row i, 256 queries): the query side from z (LN, q
//                  for the 4 heads), online-softmax attention over all keys,
//                  and in the epilogue the gate (LN, g), the output projection
//                  and the residual, added in place.  q and g never leave the
//                  chip.
// H = 4 heads of d = 32 over c = 128 channels.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int C = 128;
constexpr int H = 4;
constexpr int DH = 32;
constexpr int kProjRows = 4 * C + H;       // q, k, v, g, bias rows of the packed weight
constexpr int kRowQ = 0, kRowK = C, kRowG = 3 * C, kRowB = 4 * C;   // first rows of q, k (v follows), g, bias
constexpr int kProjRowsLds = 2 * C + 32;   // k, v and the bias block (padded to 32 rows) staged by triatt_proj
constexpr int kProjThreads = 512;
constexpr int kProjSmem = kProjRowsLds * kLdw * 2 + kProjRowsLds * 2 * 2;
constexpr int kFlashThreads = 256;         // 4 waves
constexpr int kFlashTiles = 2;             // 32-query tiles per wave (1 tile at 3 waves per SIMD measured slower)
constexpr int kFlashQueries = 4 * 32 * kFlashTiles;   // queries per workgroup
constexpr int kFlashWavesPerEu = kFlashTiles == 1 ? 3 : 2;
constexpr int kMaxKeyBlocks = 16384 / 64;  // 64-key blocks of the longest row (N <= 16384)

// Softmax in base 2: q is stored pre-scaled by log2(e)/sqrt(d) and the bias by
// log2(e), so QK^T + bias comes out of the MFMA directly in log2 units.
constexpr float kQScale = 0.17677669529663687f * kLog2e;

struct TriAttBuffers {
  bf16* k;       // [B][Np][H][Np][DH]  per frame row and head: keys x head channels
  bf16* vt;      // [B][Np][C][Np]  channel-major per frame row
  bf16* bias;    // [B][H][Np/32][Np/64][4][64][8]  times log2(e), in MFMA B-operand tiles
                 //   (see bias_tile_index)
  uint8_t* mask; // [B][Np][Np]     frame-ordered 0/1 (0 outside [0, N))
};

// Bias storage: for head h, query q and key k the value sits in the 4 KB tile
// (h, q / 32, k / 64) at chunk x = (k % 64) / 16, lane (q % 32) + 32 ((k % 16) / 8),
// element k % 8 -- the B-operand layout in which the attention kernel adds the
// bias, so that each of its bias loads is 1 KB contiguous.  For k a multiple of
// 8 this returns the start of the 8-key chunk.
__device__ __forceinline__ size_t bias_tile_index(int h, int q, int k, int Np) {
  const size_t tile = ((size_t)h * (Np / 32) + q / 32) * (Np / 64) + k / 64;
  const int x = (k & 63) >> 4, lane = (q & 31) + 32 * ((k & 15) >> 3);
  return tile * 2048 + (x * 64 + lane) * 8 + (k & 7);
}

// ---------------------------------------------------------------------------
// Projection kernel.  Tile = (b, frame row i, 32 frame columns).
// ---------------------------------------------------------------------------
template <bool kStarting>
__global__ __launch_bounds__(kProjThreads) void triatt_proj_kernel(
    const bf16* __restrict__ z, const uint8_t* __restrict__ mask, const bf16* __restrict__ wf,
    const bf16* __restrict__ cf, TriAttBuffers buf, int B, int N, int Np) {
  // LDS rows: k (0 .. C-1), v (C .. 2C-1), bias (2C .. 2C+H-1, zero-padded to 32 rows).
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  bf16* cl = wl + kProjRowsLds * kLdw;
  stage_weights(wl, wf + (size_t)kRowK * C, 2 * C, 2 * C);
  stage_weights(wl + 2 * C * kLdw, wf + (size_t)kRowB * C, H, 32);
  stage_bias(cl, cf + 2 * kRowK, 2 * C, 2 * C);
  stage_bias(cl + 2 * 2 * C, cf + 2 * kRowB, H, 32);
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rho = lane & 31, h = lane >> 5;
  const int waves = blockDim.x >> 6;
  const unsigned tiles_per_row = Np / 32;
  const unsigned ntiles = (unsigned)B * Np * tiles_per_row;
  const size_t plane = (size_t)Np * Np;

  // Software pipeline over this wave's tiles: tile t + stride's inputs (this
  // lane's half of the z row of its pair slot and the mask byte of frame
  // column k0 + rho) are loaded before tile t's stores are issued and
  // normalised after them.  Vector-memory counters retire in issue order, so
  // waiting for those loads then does not wait for the stores to be written,
  // and, being in straight-line code, the wait the compiler places is exact.
  const unsigned stride = gridDim.x * waves;
  bf16x8 raw[8];
  uint8_t mraw = 0;
  bool mok = false;
  auto fetch = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tiles_per_row, Np);
    const int i = ti.row, b = ti.b, k0 = ti.col * 32;
    const int kc = k0 + rho, kk = k0 + perm32(rho);
    mok = i < N && kc < N;
    const size_t mp = !mok ? 0 : kStarting ? ((size_t)b * N + i) * N + kc : ((size_t)b * N + kc) * N + i;
    mraw = mask[mp];
    // Unconditional loads (pair 0 for slots outside the sequence, zeroed in
    // prepare): a zero-filled destination would be written before the loads,
    // and overwriting registers that earlier stores read makes the compiler
    // wait for those stores.
    const bool valid = i < N && kk < N;
    const size_t zpair = !valid ? 0 : kStarting ? ((size_t)b * N + i) * N + kk : ((size_t)b * N + kk) * N + i;
    const bf16* row = z + zpair * C + 8 * h;
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) raw[s8] = load8(row + 16 * s8);
  };
  // Tile operands: normalised row x, the bias k-step operand xb and the mask byte.
  bf16x8 x[8], xb;
  uint8_t mv;
  auto prepare = [&](unsigned tt) {
    const TileIdx ti = split_tile(tt, tiles_per_row, Np);
    const int kk = ti.col * 32 + perm32(rho);
    const bool valid = ti.row < N && kk < N;
    float v[64];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) unpack8(valid ? raw[s8] : bf16x8{}, v + 8 * s8);
    normalize_half_row(v, valid, x);
    xb = bias_step_x(valid, h);
    mv = mok && mraw != 0;
  };

  unsigned t = blockIdx.x * waves + wave;
  if (t < ntiles) {
    fetch(t);
    prepare(t);
  }
  for (; t < ntiles; t += stride) {
    const unsigned tn = t + stride;
    if (tn < ntiles) fetch(tn);
    const TileIdx ti = split_tile(t, tiles_per_row, Np);
    const int kt = ti.col, i = ti.row, b = ti.b;
    const int k0 = kt * 32;
    // This lane's pair slot: frame (i, k0 + perm32(rho)).
    const int kk = k0 + perm32(rho);

    const size_t frow = ((size_t)b * Np + i) * Np;  // frame row base (pairs)
    // Frame rows past N: the attention kernel reads only their bias (the
    // bias row of query i, used by waves whose queries straddle N) and mask.
    if (i < N) {
      // k: head-major per frame row, [H][Np][DH]; lane holds pair slot
      // perm32(rho), head cb's channels 16h .. 16h + 15.
#pragma unroll 1
      for (int cb = 0; cb < 4; ++cb) {
        const f32x16 a = proj_block_pm_f(x, xb, wl, cl, cb * 32, rho, h);
        float vk[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) vk[u] = a[u];
        store16(buf.k + (frow * H + (size_t)cb * Np + kk) * DH + 16 * h, vk);
      }
      // v^T: channel-major.  Lane (n, h) holds channel cb*32+n, pairs k0+16h..+15.
#pragma unroll 1
      for (int cb = 0; cb < 4; ++cb) {
        const f32x16 av = proj_block_cm_f(x, xb, wl, cl, C + cb * 32, rho, h);
        float vv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) vv[u] = av[u];
        store16(buf.vt + (((size_t)b * Np + i) * C + cb * 32 + rho) * Np + k0 + 16 * h, vv);
      }
    }
    {
      const f32x16 ab = proj_block_cm_f(x, xb, wl, cl, 2 * C, rho, h);
      if (rho < H) {
        float vb[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) vb[u] = ab[u] * kLog2e;
        // keys k0 + 16h + u: u < 8 and u >= 8 go to the chunks of lanes hh = 0 / 1
        bf16* dst = buf.bias + (size_t)b * H * plane + bias_tile_index(rho, i, k0 + 16 * h, Np);
        bf16x8 lo, hi;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          lo[u] = f2bf(vb[u]);
          hi[u] = f2bf(vb[8 + u]);
        }
        store8(dst, lo);
        store8(dst + 32 * 8, hi);
      }
    }
    if (h == 0) buf.mask[frow + k0 + rho] = mv;
    if (tn < ntiles) prepare(tn);
  }
}

// ---------------------------------------------------------------------------
// Weights of the attention kernel's own projections in MFMA A-operand
// fragment order: fragment f of 32 weight rows x 16 inputs is 1 KB contiguous
// (lane l at bytes 16 l), so each fragment load reads whole cache lines.
//   f = 0 .. 31   q rows, LayerNorm gamma folded in: block hd = f / 8, k-step
//                 s = f % 8, lane (n, hh) holds W'q[hd*32 + perm32(n)][16 s + 8 hh + 0..7]
//   f = 32 .. 63  g rows, folded: W'g[hd*32 + perm32(n)][32 (s >> 1) + 16 hh + 8 (s & 1) + 0..7]
//   f = 64 .. 95  Wo: Wo[cb*32 + perm32(n)][32 (s >> 1) + 16 hh + 8 (s & 1) + 0..7]
// The folded values are W * gamma rounded to bf16, bit for bit the fold of the
// projection rows.
// ---------------------------------------------------------------------------
constexpr int kFragCount = 96;
constexpr int kFragElems = kFragCount * 64 * 8;

__global__ __launch_bounds__(256) void triatt_frag_kernel(const bf16* __restrict__ w_proj,
                                                          const float* __restrict__ gamma,
                                                          const bf16* __restrict__ w_o, bf16* __restrict__ wt) {
  const int slot = blockIdx.x * 256 + threadIdx.x;   // 16-byte slot
  if (slot >= kFragCount * 64) return;
  const int f = slot >> 6, lane = slot & 63, n = lane & 31, hh = lane >> 5;
  const int kind = f >> 5, blk = (f >> 3) & 3, s = f & 7;
  const int row = blk * 32 + perm32(n);
  const int c0 = kind == 0 ? 16 * s + 8 * hh : 32 * (s >> 1) + 16 * hh + 8 * (s & 1);
  const bf16* src = kind == 2 ? w_o + (size_t)row * C : w_proj + (size_t)((kind == 0 ? kRowQ : kRowG) + row) * C;
  const bf16x8 w = load8(src + c0);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = kind == 2 ? w[e] : f2bf(bf2f(w[e]) * gamma[c0 + e]);
  store8(wt + (size_t)slot * 8, o);
}

// ---------------------------------------------------------------------------
// Flash attention kernel.  Workgroup = (b, frame row i, 256 queries); wave w
// owns the kFlashTiles = 2 32-query tiles q0 and q0 + 32, q0 = 256 qb + 64 w,
// which share every K / V fragment the wave reads from LDS.
//
// Query side and gate in the kernel: the prologue reads the z rows of the
// wave's queries, normalises them and projects q for the four heads on MFMA
// (head 0's into registers, the others into LDS slots); the epilogue reads the
// same rows again for the residual and projects the gate g from them.  Only
// the keys, values, bias and mask come from the projection kernel.
//
// Rows whose keys are all masked take a closed form (uniform weights: o / l is
// the mean of v), and 64-key blocks without a valid key are skipped: their
// logits (-1e30 or -inf) add exact zeros, so o and l are bit-identical.
//
// At head dim 32 the attention is bound by vector-ALU and issue work, not by
// the matrix cores, so everything that can ride on an MFMA does:
//   S^T = K Q^T               2 MFMAs (k-steps over d)
//       + bias               2 MFMAs: A = one-hot "identity" fragments,
//                             B = the bias tile in B-operand layout
//       + key mask - m       1 MFMA:  rank-2 product of a per-key column
//                             (0 valid, -1e30 masked, -inf beyond N) and a
//                             column of ones with (1, -m); skipped for a block
//                             without masked keys while no shift is in use
// A masked key's logit is -1e30 + (q.k + bias) = -1e30 exactly in fp32, so a
// fully masked row gets equal logits (uniform weights, the reference's
// masked_fill(-1e6) result) and a partially masked row gets exact zeros.
// Softmax shift: when the first block's row maxima all lie in [-64, 16] (log2
// units) the logits enter exp2 unshifted; otherwise the running max m is set
// from that block.  After the first block, m is only set or moved (o and l
// rescaled) when a block's weight sum exceeds 2^16 (a weight above 2^16 may be
// present), so most blocks skip the max search.
//
// Loops: heads outermost (one head's accumulator live; a finished head parks
// o/l as bf16 in the LDS slot its successor's q has just left, the last
// head's stays in registers), then 64-key blocks.  A block is two
// independent 32-key halves whose MFMA chains and softmax interleave.  The 4
// waves share frame row i, so each (head, 64-key) tile of K and V^T is staged
// once per workgroup in LDS, double-buffered; the next tile and the next
// bias slice are fetched while the current block is consumed.
//
// Layouts: q fragments lane (n, hh) <-> channels 16hh .. 16hh + 15 of query
// q0 + n (k-step j: 8 of them, against K chunk 2hh + j); S^T D lane (n, hh)
// register u <-> key k0 + 16hh + u of query q0+n (A rows = keys
// k0 + perm32(rho)); O^T = V^T P^T with P^T taken straight
// from the softmax registers (k-step s, half hh, t <-> key k0 + 16hh + 8s + t),
// D lane (n, hh) register u <-> d = 16hh + u; the epilogue feeds g*o back as
// the B operand of update^T = Wo (g*o)^T.  LDS tiles are [32][32] bf16,
// unpadded 64-byte rows whose 16-byte chunk index is XORed with row bits 2
// and 3: the perm32-row operand reads and the staging writes (each wave writes
// one contiguous 1 KB: 16 rows x 4 chunks) are free of bank conflicts on
// gfx950 (measured with SQ_LDS_BANK_CONFLICT).
// ---------------------------------------------------------------------------
constexpr int TLD = 32;                 // LDS row stride (bf16) of a [32][32] tile
constexpr int kTile = 32 * TLD;
constexpr int kStage = 4 * kTile;       // K (2 halves) + V^T (2 halves)
constexpr float kSlackSum = 65536.0f;   // 2^16: a block sum above this may hold p > 2^16

__device__ __forceinline__ int t_off(int r, int chunk) { return r * TLD + ((chunk ^ ((r >> 2) & 3)) << 3); }

// With kTail the residual stream z carries an int8 tail plane (common.h),
// read with z and rewritten with out (in place).
// wt: the q and g rows of the packed projection (LayerNorm folded in) and Wo
// in fragment order (triatt_frag_kernel); cf: the folded projection's bias
// pairs (fold.hip), of which this kernel uses the q and g rows; z is read for the query side, the gate and the residual (z = zres;
// out may alias it: every workgroup reads and writes only its own pairs).
template <bool kStarting, bool kTail>
__global__ __launch_bounds__(kFlashThreads) __attribute__((amdgpu_waves_per_eu(kFlashWavesPerEu, kFlashWavesPerEu)))
void triatt_flash_kernel(
    TriAttBuffers buf, const bf16* __restrict__ wt, const bf16* __restrict__ cf,
    const bf16* zres, bf16* out, int8_t* tail, int N, int Np, int residual, int nitems) {
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kStage];
  // H - 1 slots of [kFlashQueries][DH] bf16: slot s holds q of head s + 1 (times
  // kQScale) until that head starts, then o / l of head s until the epilogue
  // (head 0's q goes straight to registers, head H-1's o / l stays in them).
  // A lane reads and writes only its own 32 bytes of a slot.
  __shared__ __attribute__((aligned(16))) bf16 qo[(H - 1) * kFlashQueries * DH];
  extern __shared__ __attribute__((aligned(16))) bf16 kadd[];   // [Np] additive key mask
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  // XCD-aware mapping: workgroup w runs on XCD w % 8.  Frame rows (b, i)
  // are dealt to the XCDs round-robin (row r to XCD r % 8) and each XCD runs
  // a row's query blocks one after another, so the blocks of a row (which read
  // the same K and V) share an L2, and rows of every kind (padded rows are
  // nearly free) spread evenly over the XCDs.
  const int nq = (Np + kFlashQueries - 1) / kFlashQueries;
  const int xcd = blockIdx.x % 8, local = blockIdx.x / 8;
  const int row = (local / nq) * 8 + xcd;   // b * N + i
  if (row >= nitems / nq) return;           // before any barrier: the whole workgroup leaves
  const int qb = local % nq;
  const int i = row % N;
  const int b = row / N;
  // This wave's 32-query tiles: q0 + 32t (Np is a multiple of 64, so all of
  // them exist or none does).
  const int q0 = qb * kFlashQueries + wave * 32 * kFlashTiles;
  const bool active = q0 < Np;
  // A wave none of whose queries lies in [0, N) has nothing to store: it
  // still stages tiles, fetches operands and meets every barrier, but skips
  // the matrix products and the softmax (the operand fetches stay, so the
  // memory-counter waits of both kinds of wave are the same).
  const bool compute = q0 < N;
  int qrow[kFlashTiles];
#pragma unroll
  for (int t = 0; t < kFlashTiles; ++t) qrow[t] = active ? q0 + 32 * t + n : 0;
  // This lane's 16 channels (16 hh .. 16 hh + 15) of query q0 + 32 t + n in LDS slot sl
  auto slot_at = [&](int sl, int t) {
    return qo + ((size_t)sl * kFlashQueries + wave * 32 * kFlashTiles + 32 * t + n) * DH + 16 * hh;
  };
  bf16x8 olast[kFlashTiles][2];   // o / l of the last head

  const size_t frow = ((size_t)b * Np + i) * Np;
  const unsigned plane = (unsigned)Np * (unsigned)Np;

  const bf16* __restrict__ kg = buf.k + frow * C;                           // [H][Np keys][DH]
  const bf16* __restrict__ vg = buf.vt + ((size_t)b * Np + i) * C * Np;     // [C][Np keys]
  const bf16* __restrict__ bg = buf.bias + (size_t)b * H * plane;           // [H][Np][Np]
  // z pair of frame pair (i, q) (pair 0 for q >= N: read, never stored)
  auto zpair_of = [&](int q) -> size_t {
    return q >= N ? 0 : kStarting ? ((size_t)b * N + i) * N + q : ((size_t)b * N + q) * N + i;
  };
  // q fragments of the head being processed: lane (n, hh) holds channels
  // 16 hh .. 16 hh + 15 of query q0 + 32 t + n (as the K fragments pair them:
  // k-step 0 <-> K chunk 2 hh, k-step 1 <-> K chunk 2 hh + 1).  Head 0's come
  // from the prologue, each later head's from its LDS slot during the
  // previous head's last key block.
  bf16x8 qf[kFlashTiles][2];
  auto qload = [&](int hq) {
#pragma unroll
    for (int t = 0; t < kFlashTiles; ++t) {
      qf[t][0] = load8(slot_at(hq - 1, t));
      qf[t][1] = load8(slot_at(hq - 1, t) + 8);
    }
  };
  // Key-mask row (additive: 0 valid, -1e30 masked, -inf beyond N).  A row
  // whose keys are all masked ("dead") attends uniformly to its N keys
  // (every logit replaced by the same value): o / l is the mean of v.
  // One pass over the mask row also flags the 64-key blocks holding a valid
  // key (wave w covers keys [256 j + 64 w, +64): block 4 j + w; Np is a
  // multiple of 64, so the trip count is the same for the 64 lanes).
  __shared__ uint8_t kflag[kMaxKeyBlocks];
  int any_valid = 0;
  for (int t = tid; t < Np; t += kFlashThreads) {
    const bool valid = t < N && buf.mask[frow + t] != 0;
    any_valid |= valid;
    kadd[t] = f2bf(valid ? 0.f : t >= N ? -INFINITY : -1e30f);
    const bool any_ok = __any(valid);
    if (lane == 0) kflag[t >> 6] = any_ok;
  }
  const bool dead = __syncthreads_or(any_valid) == 0;

  // Operand fetches through buffer resources: per-lane byte offsets are fixed,
  // the (head, key block) part is a wave-uniform scalar offset.
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kg, (unsigned)Np * C * 2);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(vg, (unsigned)Np * C * 2);
  const __amdgpu_buffer_rsrc_t brs = buffer_rsrc(bg, (unsigned)H * plane * 2);

  // Staging of one (head, 64-key) tile: K is 64 key rows x 4 chunks (two
  // 32-key halves), V^T two 32-key halves of 32 d rows x 4 chunks; thread tid
  // moves K chunk tid and, in V^T half tid >> 7, row (tid >> 2) & 31, chunk
  // tid & 3, so every wave writes one contiguous 1 KB of each.
  const int k_row = tid >> 2, k_chunk = tid & 3;
  const int v_half = tid >> 7, v_row = (tid >> 2) & 31, v_chunk = tid & 3;
  const unsigned k_voff = (unsigned)tid * 16;   // = (k_row * DH + k_chunk * 8) * 2
  const unsigned v_voff = ((unsigned)v_row * Np + 32 * v_half + v_chunk * 8) * 2;
  const int k_lds = (k_row >> 5) * kTile + t_off(k_row & 31, k_chunk);
  const int v_lds = 2 * kTile + v_half * kTile + t_off(v_row, v_chunk);
  bf16x8 rk, rv;
  auto gload = [&](int hn, int kn) {
    rk = buffer_load8(krs, k_voff, (unsigned)(hn * Np + kn) * DH * 2);
    rv = buffer_load8(vrs, v_voff, (unsigned)(hn * DH * Np + kn) * 2);
  };
  auto lstore = [&](int st) {
    store8(smem + st * kStage + k_lds, rk);
    store8(smem + st * kStage + v_lds, rv);
  };
  // Bias slices in B-operand layout: lane (n, hh), half a, k-step s <-> keys
  // k0 + 32a + 16s + 8hh + t.  One tile's bias slice for a (head, 64-key)
  // block is one contiguous 4 KB: instruction x reads 1 KB, lane l at byte 16 l.
  const unsigned bias_voff = (unsigned)lane * 16;
  auto bload = [&](int hn, int kn, int t, bf16x8 (&bb)[4]) {
    const unsigned soff = (unsigned)bias_tile_index(hn, active ? q0 + 32 * t : 0, kn, Np) * 2;
#pragma unroll
    for (int x = 0; x < 4; ++x) bb[x] = buffer_load8(brs, bias_voff + 1024 * x, soff);
  };

  const int krow = perm32(n);
  // One-hot fragments: A[rho][(s, hh, t)] = 1 iff perm32(rho) == 16s + 8hh + t.
  bf16x8 ident[2], zero8;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    ident[0][t] = f2bf(krow == 8 * hh + t ? 1.f : 0.f);
    ident[1][t] = f2bf(krow == 16 + 8 * hh + t ? 1.f : 0.f);
    zero8[t] = f2bf(0.f);
  }

  if (dead) {
    // Uniform weights over the N keys: o / l = mean of v (v is exactly 0 for
    // keys in [N, Np)), the same for every query of the row.
    float* vmean = reinterpret_cast<float*>(smem);
    constexpr int kWaves = kFlashThreads / 64, kChan = 8;   // channels whose loads are in flight together
    for (int c0 = wave; c0 < C; c0 += kChan * kWaves) {
      float acc[kChan];
#pragma unroll
      for (int j = 0; j < kChan; ++j) acc[j] = 0.f;
      for (int k = lane * 8; k < Np; k += 512) {
        bf16x8 x[kChan];
#pragma unroll
        for (int j = 0; j < kChan; ++j) x[j] = load8(vg + (size_t)(c0 + kWaves * j) * Np + k);
#pragma unroll
        for (int j = 0; j < kChan; ++j) {
          float v8[8];
          unpack8(x[j], v8);
#pragma unroll
          for (int u = 0; u < 8; ++u) acc[j] += v8[u];
        }
      }
#pragma unroll
      for (int j = 0; j < kChan; ++j) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc[j] += __shfl_xor(acc[j], off);
        if (lane == 0) vmean[c0 + kWaves * j] = acc[j] * (1.0f / N);
      }
    }
    __syncthreads();
#pragma unroll
    for (int hd = 0; hd < H; ++hd) {
      bf16x8 r[2];
#pragma unroll
      for (int u = 0; u < 16; ++u) r[u >> 3][u & 7] = f2bf(vmean[hd * DH + 16 * hh + u]);
#pragma unroll
      for (int t = 0; t < kFlashTiles; ++t) {
        if (hd + 1 < H) {
          store8(slot_at(hd, t), r[0]);
          store8(slot_at(hd, t) + 8, r[1]);
        } else {
          olast[t][0] = r[0];
          olast[t][1] = r[1];
        }
      }
    }
  } else {
  if (compute) {
    // Query side: LN(z) (affine-free; gamma and beta are folded into the q
    // rows of wf / cf) and q = LN(z) Wq^T * kQScale for the four heads, on
    // MFMA with the weight rows as the A operand (pair-major blocks: lane
    // (n, hh) ends with query n's channels 16 hh + u).  A query past N has a
    // zero row and q = 0, as the reference's padded pairs project to.
    bf16x8 xq[kFlashTiles][8], xbq[kFlashTiles];
#pragma unroll
    for (int t = 0; t < kFlashTiles; ++t) {
      const int q = q0 + 32 * t + n;
      float v[64];
      load_half_row_f32(zres + zpair_of(q) * C, hh, true, v);
      normalize_half_row(v, q < N, xq[t]);
      xbq[t] = bias_step_x(q < N, hh);
    }
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wt, (unsigned)kFragElems * 2);
#pragma unroll 1
    for (int hd = 0; hd < H; ++hd) {
      const int r = kRowQ + hd * DH + perm32(n);
      bf16x8 wq[8], wb = zero8;
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2)
        wq[s2] = buffer_load8(wrs, (unsigned)lane * 16, (unsigned)(hd * 8 + s2) * 1024);
      if (hh == 0) {
        wb[0] = cf[2 * r];
        wb[1] = cf[2 * r + 1];
      }
#pragma unroll
      for (int t = 0; t < kFlashTiles; ++t) {
        f32x16 acc = zero16();
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) acc = mfma32(wq[s2], xq[t][s2], acc);
        acc = mfma32(wb, xbq[t], acc);
        bf16x8 r0, r1;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          r0[u] = f2bf(acc[u] * kQScale);
          r1[u] = f2bf(acc[8 + u] * kQScale);
        }
        if (hd == 0) {
          qf[t][0] = r0;
          qf[t][1] = r1;
        } else {
          store8(slot_at(hd - 1, t), r0);
          store8(slot_at(hd - 1, t) + 8, r1);
        }
      }
    }
  }
  // Key blocks with at least one valid key, in order.  A block whose keys are
  // all masked adds exact zeros (its logits are -1e30 or -inf below any
  // unmasked logit), so skipping it leaves o and l bit-identical.
  __shared__ short act[kMaxKeyBlocks];
  __shared__ int nact_s;
  const int nk = Np / 64;
  if (wave == 0) {
    int base = 0;
    for (int c0 = 0; c0 < nk; c0 += 64) {
      const int kb = c0 + lane;
      const bool f = kb < nk && kflag[kb] != 0;
      const unsigned long long bal = __ballot(f);
      if (f) act[base + __popcll(bal & ((1ull << lane) - 1ull))] = (short)kb;
      base += __popcll(bal);
    }
    if (lane == 0) nact_s = base;
  }
  __syncthreads();
  const int nact = nact_s;   // >= 1: the row has a valid key
  bf16x8 bias[kFlashTiles][4];   // per query tile: bias slice of the block being consumed, then of the next one

  gload(0, act[0] * 64);
#pragma unroll
  for (int t = 0; t < kFlashTiles; ++t) bload(0, act[0] * 64, t, bias[t]);
  lstore(0);
  __syncthreads();
  int st = 0;
  bf16 kma = kadd[act[0] * 64 + krow], kmb = kadd[act[0] * 64 + 32 + krow];   // key-mask column of the block consumed next
#pragma unroll 1
  for (int hd = 0; hd < H; ++hd) {
    f32x16 o[kFlashTiles];
    float m[kFlashTiles], l[kFlashTiles];
    // Per tile, three modes: fresh (no block consumed), unshifted (the
    // logits enter exp2 as they are: the first block's maxima were all in
    // [-64, 16]) and shifted (m_set: the MFMA subtracts m, the bf16-rounded
    // max of some unmasked logit).
    bool m_set[kFlashTiles], fresh[kFlashTiles];
#pragma unroll
    for (int t = 0; t < kFlashTiles; ++t) {
      o[t] = zero16();
      m[t] = -INFINITY;
      l[t] = 0.f;
      m_set[t] = false;
      fresh[t] = true;
    }
    // B operand of the rank-2 mask / shift product: k = 0 -> 1 (picks the key
    // column kadd), k = 1 -> -m (against a key column of ones).
    bf16x8 qm[kFlashTiles];
#pragma unroll
    for (int t = 0; t < kFlashTiles; ++t) {
      qm[t] = zero8;
      if (hh == 0) qm[t][0] = f2bf(1.f);
    }
    // One 64-key block (the ib-th active one): fetch the next K/V tile,
    // consume the current one.  k0 and the next tile's first key (kn) come in
    // registers; the key after that is read from the list during the block
    // (a read at the block's start would stall the K/V fetch on it).
    auto block = [&](int ib, int k0, int& kn, bf16& kma, bf16& kmb) {
      // next tile: the next active block of this head, else the first of the
      // next head; the very last iteration refetches itself
      const int hn = ib + 1 < nact || hd + 1 == H ? hd : hd + 1;
      gload(hn, kn);
      const int ia = ib + 2 < nact ? ib + 2 : ib + 2 - nact;    // block after the next (wraps to the next head)
      const int kafter = act[ia < nact ? ia : 0] * 64;
      // Every wave runs the block, idle ones (q0 >= Np, only when Np is not a
      // multiple of 256) on row 0 queries whose results they never store: with
      // a branch here the compiler's wait before the K / V staging store below
      // would have to cover the inactive path too, where nothing follows the
      // K / V loads, and would then also wait for the bias prefetch.
      {
        const bf16* ks = smem + st * kStage;
        const bf16* vs = ks + 2 * kTile;
        // the key-mask column matters only for a block holding a masked key
        const bool need_mask = __any(bf2f(kma) != 0.f || bf2f(kmb) != 0.f);
        bf16x8 km0 = zero8, km1 = zero8;
        if (hh == 0) {
          km0[0] = kma;
          km1[0] = kmb;
          km0[1] = f2bf(1.f);
          km1[1] = f2bf(1.f);
        }
        // the next block's key-mask column, read now so the read is not waited on at its start
        kma = kadd[kn + krow];
        kmb = kadd[kn + 32 + krow];
        const bf16x8 ka0 = load8(ks + t_off(krow, 2 * hh)), ka1 = load8(ks + kTile + t_off(krow, 2 * hh));
        const bf16x8 kb0 = load8(ks + t_off(krow, 2 * hh + 1)), kb1 = load8(ks + kTile + t_off(krow, 2 * hh + 1));
        // Logits minus the running max m, all on MFMA (no shift unless m is
        // set; the rank-2 product only when there is a mask or a shift).
        //
        // Instruction order.  This chip overlaps a wave's VALU work with its
        // own MFMAs in flight, not with another wave's, so the block is laid
        // out as segments fenced by sched_barrier, each pairing MFMAs with
        // independent VALU work of the same wave:
        //   A: tile 0's logit MFMAs;
        //   B: tile 1's logit MFMAs, each with a share of tile 0's weights
        //      (exp2 of the logits as they are: the fast path, computed before
        //      it is known to apply and recomputed by the slow path if not);
        //   C: tile 0's P.V MFMAs with a share of tile 1's weights;
        //   D: tile 1's P.V MFMAs.
        static_assert(kFlashTiles == 2, "the segment layout pairs two query tiles");
        f32x16 s[kFlashTiles][2];
        bf16x8 pa[kFlashTiles][2], pb[kFlashTiles][2];
        // the j-th logit MFMA of tile t (0-3: q.k, 4-7: bias)
        auto logit_mfma = [&](int t, int j) {
          switch (j) {
            case 0: s[t][0] = mfma32(ka0, qf[t][0], zero16()); break;
            case 1: s[t][1] = mfma32(ka1, qf[t][0], zero16()); break;
            case 2: s[t][0] = mfma32(kb0, qf[t][1], s[t][0]); break;
            case 3: s[t][1] = mfma32(kb1, qf[t][1], s[t][1]); break;
            case 4: s[t][0] = mfma32(ident[0], bias[t][0], s[t][0]); break;
            case 5: s[t][1] = mfma32(ident[0], bias[t][2], s[t][1]); break;
            case 6: s[t][0] = mfma32(ident[1], bias[t][1], s[t][0]); break;
            default: s[t][1] = mfma32(ident[1], bias[t][3], s[t][1]); break;
          }
        };
        auto mask_shift = [&](int t) {
          if (m_set[t] || need_mask) {
            bf16x8 qs = qm[t];
            if (!m_set[t]) qs[1] = f2bf(0.f);
            s[t][0] = mfma32(km0, qs, s[t][0]);
            s[t][1] = mfma32(km1, qs, s[t][1]);
          }
        };
        // fast-path weights of tile t, part j of 8: four values of pa (j < 4) or
        // pb.  The empty asm pins them to this segment (left alone, the
        // optimizer sinks the pure exponentials to their first use).
        auto exp_part = [&](int t, int j) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int u = 4 * (j & 3) + e;
            if (j < 4)
              pa[t][u >> 3][u & 7] = f2bf(fast_exp2(s[t][0][u]));
            else
              pb[t][u >> 3][u & 7] = f2bf(fast_exp2(s[t][1][u]));
          }
          bf16x8& done = j < 4 ? pa[t][(j & 3) >> 1] : pb[t][(j & 3) >> 1];
          asm volatile("" : "+v"(done));
        };
        bf16x8 vf[4];   // V^T fragments of the block (shared by both tiles)
        auto pv_mfma = [&](int t, int j) {
          o[t] = mfma32(vf[j], j < 2 ? pa[t][j & 1] : pb[t][j & 1], o[t]);
        };
        // Weight sum of tile t; a block sum above 2^16 may hold a weight above
        // 2^16 (then m moves: rare), and a fresh tile has no shift yet: both
        // take the slow path, which recomputes the weights.
        auto finish = [&](int t) {
          f32x16& s0 = s[t][0];
          f32x16& s1 = s[t][1];
          float psum = sum8_bf16(pa[t][1], sum8_bf16(pa[t][0], 0.f)) + sum8_bf16(pb[t][1], sum8_bf16(pb[t][0], 0.f));
          if (fresh[t] || __any(psum > kSlackSum)) {
            // s0, s1 hold the logits minus `shift` (the MFMA subtracts m
            // once m is set).  Everything here works on those shifted values,
            // so the fast path never needs the unshifted logits.
            const float shift = m_set[t] ? m[t] : 0.f;
            float bmax = fmaxf(s0[0], s1[0]);
#pragma unroll
            for (int u = 1; u < 16; ++u) bmax = __builtin_fmaxf(bmax, __builtin_fmaxf(s0[u], s1[u]));
            bmax = fmaxf(bmax, __shfl_xor(bmax, 32)) + shift;
            float delta = 0.f;
            if (fresh[t] && __all(bmax >= -64.f && bmax <= 16.f)) {
              // unshifted from here on: every weight is at most 2^16 until a
              // block sum says otherwise, and each row keeps a weight of at
              // least 2^-64 (nothing is accumulated yet)
              fresh[t] = false;
            } else {
              // The shift is kept bf16-representable: it enters the MFMA as -m.
              // Leaving the unshifted mode, the running max is at least -64.
              const float floor_m = m_set[t] ? m[t] : fresh[t] ? -INFINITY : -64.f;
              const float m_new = bf2f(f2bf(fmaxf(floor_m, bmax)));
              const float alpha = fresh[t] ? 0.f : fast_exp2(shift - m_new);
              delta = m_new - shift;
              m[t] = m_new;
              l[t] *= alpha;
#pragma unroll
              for (int u = 0; u < 16; ++u) o[t][u] *= alpha;
              // a block of masked keys only (logits ~ -1e30) does not set m
              m_set[t] = m_set[t] || __all(m[t] > -1e29f);
              fresh[t] = fresh[t] && !m_set[t];
              if (hh == 0) qm[t][1] = f2bf(-m[t]);
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
              pa[t][u >> 3][u & 7] = f2bf(fast_exp2(s0[u] - delta));
              pb[t][u >> 3][u & 7] = f2bf(fast_exp2(s1[u] - delta));
            }
            psum = sum8_bf16(pa[t][1], sum8_bf16(pa[t][0], 0.f)) + sum8_bf16(pb[t][1], sum8_bf16(pb[t][0], 0.f));
          }
          l[t] += psum;
        };
        if (compute) {
          // A
#pragma unroll
          for (int j = 0; j < 8; ++j) logit_mfma(0, j);
          mask_shift(0);
        }
        bload(hn, kn, 0, bias[0]);
        if (compute) {
          // B
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            logit_mfma(1, j);
            exp_part(0, j);
            if (j == 7) {
              vf[0] = load8(vs + t_off(krow, 2 * hh));
              vf[1] = load8(vs + t_off(krow, 2 * hh + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          mask_shift(1);
        }
        bload(hn, kn, 1, bias[1]);
        if (ib + 1 == nact && hd + 1 < H) qload(hd + 1);
        if (compute) {
          finish(0);
          // C
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (j == 0) {
              vf[2] = load8(vs + kTile + t_off(krow, 2 * hh));
              vf[3] = load8(vs + kTile + t_off(krow, 2 * hh + 1));
            }
            if ((j & 1) == 0) pv_mfma(0, j >> 1);
            exp_part(1, j);
            __builtin_amdgcn_sched_barrier(0);
          }
          finish(1);
          // D
#pragma unroll
          for (int j = 0; j < 4; ++j) pv_mfma(1, j);
        }
      }
      lstore(st ^ 1);
      st ^= 1;
      __syncthreads();
      kn = (ib + 2 < nact || hd + 1 < H) ? kafter : kn;
    };
    int kcur = act[0] * 64, knext = nact > 1 ? act[1] * 64 : (hd + 1 < H ? kcur : kcur);
#pragma unroll 1
    for (int ib = 0; ib < nact; ++ib) {
      const int k = kcur;
      kcur = knext;
      block(ib, k, knext, kma, kmb);
    }
    // head finished: o / l (bf16) parked in LDS, the last head's kept in registers
#pragma unroll
    for (int t = 0; t < kFlashTiles; ++t) {
      const float inv = 1.0f / (l[t] + __shfl_xor(l[t], 32));
      bf16x8 r[2];
#pragma unroll
      for (int u = 0; u < 16; ++u) r[u >> 3][u & 7] = f2bf(o[t][u] * inv);
      olast[t][0] = r[0];
      olast[t][1] = r[1];
      if (hd + 1 < H && compute) {
        store8(slot_at(hd, t), r[0]);
        store8(slot_at(hd, t) + 8, r[1]);
      }
    }
  }
  }
  if (!compute) return;

  // Epilogue, per 32-query tile.  Lane (n, hh) loads the z row of query
  // q0 + 32 t + n in the update's layout (channels 32 cb + 16 hh + 0..15,
  // cb = 0..3): the residual, and normalised (affine-free, gamma and beta
  // folded into the g rows of the fragment copy / cf) the gate's input, whose
  // k-step s2 = 2 cb + j carries channels 32 cb + 16 h + 8 j + e on both
  // operands.  g = sigmoid(LN(z) Wg^T) times o / l per head is the B operand
  // of update^T = Wo (g o)^T; the residual is added and the result stored in
  // z's frame.  Weight fragments (1 KB each, in fragment order: wt) are read
  // from L2 in blocks of 8 (block k = 0..3: the g rows of head k, 4..7: Wo
  // rows 32 (k - 4) ..), each block requested while the previous one is
  // multiplied; lanes of queries past N read pair 0 and store nothing.
  // One opaque copy of the weight pointer per tile: the tiles' fragments are
  // the same, and shared between the tiles (64 of them) they would not fit
  // the register budget.
  const bf16* wte[kFlashTiles];
#pragma unroll
  for (int t = 0; t < kFlashTiles; ++t) {
    wte[t] = wt;
    asm volatile("" : "+s"(wte[t]));
  }
  auto wblock = [&](int t, int k, bf16x8 (&f)[8]) {
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(wte[t], (unsigned)kFragElems * 2);
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) f[s2] = buffer_load8(r, (unsigned)lane * 16, (unsigned)(32 + 8 * k + s2) * 1024);
  };
  bf16x8 wnext[8];
  wblock(0, 0, wnext);
#pragma unroll
  for (int t = 0; t < kFlashTiles; ++t) {
    const int q = q0 + 32 * t + n;
    const bool store = q < N;
    const size_t zpair = zpair_of(q);
    bf16x8 zr[4][2];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const size_t off = zpair * C + cb * 32 + 16 * hh;
      zr[cb][0] = load8(zres + off);
      zr[cb][1] = load8(zres + off + 8);
    }
    // affine-free LayerNorm straight from the bf16 row (two-pass, fp32; no
    // fp32 copy of the row is kept, which the register budget has no room for)
    bf16x8 xg[8];
    {
      float sum = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2)
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += bf2f(zr[s2 >> 1][s2 & 1][e]);
      sum += __shfl_xor(sum, 32);
      const float mean = sum * (1.0f / C);
      float ss = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = bf2f(zr[s2 >> 1][s2 & 1][e]) - mean;
          ss += d * d;
        }
      ss += __shfl_xor(ss, 32);
      const float rstd = rsqrtf(ss * (1.0f / C) + 1e-5f);
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2)
#pragma unroll
        for (int e = 0; e < 8; ++e) xg[s2][e] = f2bf((bf2f(zr[s2 >> 1][s2 & 1][e]) - mean) * rstd);
    }
    const bf16x8 xbg = bias_step_x(true, hh);
    bf16x8 gob[2 * H];
#pragma unroll
    for (int hd = 0; hd < H; ++hd) {
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 wcur[8];
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) wcur[s2] = wnext[s2];
      wblock(t, hd + 1, wnext);
      const int r = kRowG + hd * DH + perm32(n);
      f32x16 acc = zero16();
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) acc = mfma32(wcur[s2], xg[s2], acc);
      bf16x8 wb = zero8;
      if (hh == 0) {
        wb[0] = cf[2 * r];
        wb[1] = cf[2 * r + 1];
      }
      acc = mfma32(wb, xbg, acc);
      // D lane (n, hh), register u: gate channel hd * DH + 16 hh + u of query n
      // (the last head's o / l selected, not indexed: t is a runtime index)
      const bf16x8 o0 = hd + 1 < H ? load8(slot_at(hd, t)) : t == 0 ? olast[0][0] : olast[1][0];
      const bf16x8 o1 = hd + 1 < H ? load8(slot_at(hd, t) + 8) : t == 0 ? olast[0][1] : olast[1][1];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        gob[2 * hd][u] = f2bf(sigmoidf_fast(acc[u]) * bf2f(o0[u]));
        gob[2 * hd + 1][u] = f2bf(sigmoidf_fast(acc[8 + u]) * bf2f(o1[u]));
      }
    }

    // update^T = Wo (g*o)^T (A operand: Wo row cb*32 + perm32(n), k-step s2),
    // residual add, store in z's frame.  The scheduling barrier keeps the four
    // output blocks apart (interleaved, their weight loads and accumulators
    // would not fit the register budget).
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      __builtin_amdgcn_sched_barrier(0);
      // the residual's tail, requested ahead of this block's products
      u32x4 zt;
      if (kTail) zt = load_tail16(tail + zpair * C + cb * 32 + 16 * hh);
      bf16x8 wcur[8];
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) wcur[s2] = wnext[s2];
      if (cb + 1 < 4)
        wblock(t, 5 + cb, wnext);
      else if (t + 1 < kFlashTiles)
        wblock(t + 1, 0, wnext);   // the next tile's first block
      f32x16 acc = zero16();
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) acc = mfma32(wcur[s2], gob[s2], acc);
      if (store) {
        const size_t off = zpair * C + cb * 32 + 16 * hh;
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = acc[u];
        if (kTail) {
          float zv[16];
          tail_decode16(zr[cb][0], zr[cb][1], zt, zv);
#pragma unroll
          for (int u = 0; u < 16; ++u) v[u] += zv[u];
          tail_store16(out + off, tail + off, v);
          continue;
        }
        if (residual) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            v[u] += bf2f(zr[cb][0][u]);
            v[8 + u] += bf2f(zr[cb][1][u]);
          }
        }
        store16(out + off, v);
      }
    }
  }
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

static size_t triatt_np(int64_t N) { return (size_t)round_up(N, 64); }

extern "C" size_t bioemu_triatt_workspace_bytes(int64_t B, int64_t N, int64_t Dc, int64_t Hc) {
  if (B <= 0 || N <= 0 || Dc != C || Hc != H) return 0;
  const size_t Np = triatt_np(N);
  const size_t pairs = (size_t)B * Np * Np;
  // k, v^T (bf16 x C each) + bias (bf16 x H) + mask (u8), each 256-byte aligned
  return round_up(pairs * C * 2, 256) * 2 + round_up(pairs * H * 2, 256) + round_up(pairs, 256) +
         fold_bytes(kProjRows) + (size_t)kFragElems * 2;
}

extern "C" int bioemu_triatt_fwd(const void* z, const uint8_t* mask, const float* norm_w,
                                 const float* norm_b, const void* w_proj, const void* w_o, void* out,
                                 int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t B, int64_t N,
                                 int64_t Dc, int64_t Hc, int starting, int residual,
                                 hipStream_t stream) {
  if (Dc != C || Hc != H)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "triatt: only c=128 with 4 heads of 32 is supported (got c=%lld H=%lld)",
                     (long long)Dc, (long long)Hc);
  if (res_tail && (!residual || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: res_tail needs residual=1 and 16-byte alignment");
  if (B <= 0 || N <= 0 || B > 65535 || N > 16384)
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: bad shape B=%lld N=%lld", (long long)B, (long long)N);
  if (!z || !mask || !norm_w || !norm_b || !w_proj || !w_o || !out || !workspace)
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: null pointer argument");
  if (!aligned16(z) || !aligned16(out) || !aligned16(w_proj) || !aligned16(w_o) || !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: z/out/weights/workspace must be 16-byte aligned");
  if (out == z && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: out may alias z only with residual=1");
  const size_t need = bioemu_triatt_workspace_bytes(B, N, Dc, Hc);
  if (workspace_bytes < need)
    return set_error(BIOEMU_ERR_WORKSPACE, "triatt: workspace %zu < required %zu", workspace_bytes, need);

  const int64_t Np = (int64_t)triatt_np(N);
  const size_t pairs = (size_t)B * Np * Np;
  char* p = static_cast<char*>(workspace);
  TriAttBuffers buf;
  buf.k = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * C * 2, 256);
  buf.vt = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * C * 2, 256);
  buf.bias = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * H * 2, 256);
  buf.mask = reinterpret_cast<uint8_t*>(p);
  p += round_up(pairs, 256);
  bf16* wf = reinterpret_cast<bf16*>(p);
  bf16* cf = reinterpret_cast<bf16*>(p + round_up((size_t)kProjRows * C * 2, 256));
  bf16* wt = reinterpret_cast<bf16*>(p + fold_bytes(kProjRows));
  if (B * Np * (Np / 32) >= kMaxTiles) return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: too many pair tiles");
  int rc = launch_fold_ln(w_proj, norm_w, norm_b, wf, cf, kProjRows, stream);
  if (rc) return rc;
  {
    KernelTimerScope timed("triatt_frag", stream);
    hipLaunchKernelGGL(triatt_frag_kernel, dim3(kFragCount * 64 / 256), dim3(256), 0, stream,
                       static_cast<const bf16*>(w_proj), norm_w, static_cast<const bf16*>(w_o), wt);
  }
  if ((rc = check_launch("triatt_frag"))) return rc;

  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const void* kproj = starting ? reinterpret_cast<const void*>(triatt_proj_kernel<true>)
                               : reinterpret_cast<const void*>(triatt_proj_kernel<false>);
  if (hipFuncSetAttribute(kproj, hipFuncAttributeMaxDynamicSharedMemorySize, kProjSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "triatt_proj: cannot set dynamic LDS size");
  const long long ntiles = (long long)B * Np * (Np / 32);
  const long long per_wg = kProjThreads / 64;
  const unsigned grid1 = (unsigned)std::min<long long>(cus, (ntiles + per_wg - 1) / per_wg);
  {
    KernelTimerScope timed("triatt_proj", stream);
    if (starting)
      hipLaunchKernelGGL(triatt_proj_kernel<true>, dim3(grid1), dim3(kProjThreads), kProjSmem, stream,
                         static_cast<const bf16*>(z), mask, wf, cf, buf, (int)B, (int)N, (int)Np);
    else
      hipLaunchKernelGGL(triatt_proj_kernel<false>, dim3(grid1), dim3(kProjThreads), kProjSmem, stream,
                         static_cast<const bf16*>(z), mask, wf, cf, buf, (int)B, (int)N, (int)Np);
  }
  rc = check_launch("triatt_proj");
  if (rc) return rc;

  const long long nitems = (long long)B * N * ((Np + kFlashQueries - 1) / kFlashQueries);
  const size_t flash_smem = (size_t)Np * 2;   // additive key mask row
  auto* kflash = starting ? (res_tail ? triatt_flash_kernel<true, true> : triatt_flash_kernel<true, false>)
                          : (res_tail ? triatt_flash_kernel<false, true> : triatt_flash_kernel<false, false>);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kflash), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)flash_smem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "triatt_flash: cannot set dynamic LDS size");
  const long long grid2 = ((long long)B * N + 7) / 8 * 8 * ((Np + kFlashQueries - 1) / kFlashQueries);
  if (grid2 > 0x7fffffffLL) return set_error(BIOEMU_ERR_INVALID_ARG, "triatt: too many work items");
  {
    KernelTimerScope timed("triatt_flash", stream);
    hipLaunchKernelGGL(kflash, dim3((unsigned)grid2), dim3(kFlashThreads), flash_smem, stream, buf, wt, cf,
                       static_cast<const bf16*>(z), static_cast<bf16*>(out), res_tail,
                       (int)N, (int)Np, residual, (int)nitems);
  }
  return check_launch("triatt_flash");
}
