// Row-wise Transition (SwiGLU MLP) for gfx950: the pair representation
// (c = 128) and the MSA representation (c = 64), hidden = 4c (the trunk) or
// 2c (the denoiser's pairwise conditioning, diffusion.py:498-507).
//
// Reference: Transition.forward (src/bioemu2/biomoa/ops/transition.py:52-91):
//   xn = LN(x) (eps 1e-5, with bias) when use_norm;  out = fc3(silu(fc1(xn)) * fc2(xn))
// with no biases; PairMixerLayer / Pairformer use it on z (c = 128) and
// PairMixerMSALayer on m (c = 64) (biomoa/modules/pairmixer.py:631-634).
//
// The LayerNorm affine is folded into fc1 / fc2 once per call (fold.hip):
//   LN(x) W^T = xhat (W diag(gamma))^T + W beta
// so a wave normalises its row tile affine-free and adds W beta with one
// extra MFMA k-step (pairtile.h).
//
// One workgroup = 4 waves x 32 rows.  Each wave keeps its normalised row
// tile in registers as MFMA operands and its 32 x c output accumulator in
// registers; the hidden dimension is walked in chunks of 32.  The two lanes
// (n, 0) and (n, 1) of row slot n hold alternate 8-channel chunks (lane hh
// chunk s = channels 16 s + 8 hh + 0..7), so that each 16-byte row load or
// store instruction covers 32 bytes of one cache line per row (32 lines per
// instruction rather than 64 for contiguous half rows); the fc1 / fc2 operand
// reads take weight chunk 2 s + hh to match, and the fc3 rows are staged so
// that output block cb gives lane hh the channels 32 cb + 8 hh + 0..7 and
// 32 cb + 16 + 8 hh + 0..7.  A chunk's weight
// slices (fc1 and fc2 rows, the fc3 columns and the two bias columns; 24.25 KB
// at c = 128, 12.25 KB at c = 64) are copied by buffer loads straight into LDS
// (no registers), double-buffered: chunk h + 1 is in flight while chunk h is
// multiplied.  The hidden activations never leave registers: silu(a) * b comes
// out of the fc1 / fc2 MFMAs in exactly the layout fc3 consumes as its B
// operand.
//
// LDS tiles are unpadded (the copies write 1 KB runs); the 16-byte chunk index
// of each row is XOR-swizzled so that the perm32 row pattern of the operand
// reads hits 16 distinct bank groups per 16 lanes.
#include <mutex>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int HC = 32;                      // hidden chunk
constexpr int kThreads = 256;               // 4 waves
constexpr int kRowsPerWg = 128;

template <int C, int HIDDEN>
struct Geo {
  static constexpr int HID = HIDDEN;
  static constexpr int NCH = HID / HC;                       // hidden chunks
  static constexpr int KS = C / 16;                          // 8-channel groups per lane (k-steps)
  static constexpr int RowChunks = C / 8;                    // 16-byte chunks per fc1 / fc2 row
  static constexpr int W12Tile = HC * C;                     // bf16: [32 rows][C / 8 chunks]
  static constexpr int W3Tile = C * HC;                      // bf16: [C rows][4 chunks]
  static constexpr int BiasElems = 2 * HC * 2;               // bf16: [fc1 | fc2][32 rows][hi, lo]
  static constexpr int Stage = 2 * W12Tile + W3Tile + BiasElems;
  static constexpr int Smem = 2 * Stage * 2;                 // bytes
  static constexpr int W12Copies = W12Tile * 2 / 1024;       // 1 KB copies per fc1 / fc2 tile
  static constexpr int W3Copies = W3Tile * 2 / 1024;
  static constexpr int Copies = 2 * W12Copies + W3Copies + 1;  // + the 256-byte bias copy
};

// Row swizzles of the 16-byte chunk index: 16-chunk (256 B) rows, 8-chunk
// (128 B) rows and 4-chunk (64 B) rows, each making the rows perm32(0..15)
// (and perm32(16..31)) land on distinct bank groups.
__device__ __forceinline__ int swz16(int r) { return (r & 7) | ((r & 16) >> 1); }
__device__ __forceinline__ int swz8(int r) { return ((r >> 1) & 7) ^ (((r >> 4) & 1) << 2); }
__device__ __forceinline__ int swz4(int r) { return ((r >> 2) & 1) | (((r >> 4) & 1) << 1); }
template <int C>
__device__ __forceinline__ int w12_swz(int r) { return C == 128 ? swz16(r) : swz8(r); }
template <int C>
__device__ __forceinline__ int w12_off(int r, int c) { return (r * (C / 8) + (c ^ w12_swz<C>(r))) * 8; }
__device__ __forceinline__ int w3_off(int r, int c) { return (r * 4 + (c ^ swz4(r))) * 8; }

// 16 (or 4) bytes per lane from a buffer straight into LDS at lds + 16 (4) * lane.
__device__ __forceinline__ void copy16_to_lds(__amdgpu_buffer_rsrc_t r, const bf16* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void copy4_to_lds(__amdgpu_buffer_rsrc_t r, const bf16* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 4, voff, soff, 0, 0);
}

// The residual base is res (x itself for the block's "x += T(x)"; another
// stream for "z = z_init + T(LN(z_init))").  With kTail the residual stream
// res carries an int8 tail plane (common.h), read with res and rewritten
// with out (in place).
template <int C, int HIDDEN, bool kTail>
__global__ __launch_bounds__(kThreads) void transition_rows_kernel(
    const bf16* x, const bf16* res, const bf16* __restrict__ w1, const bf16* __restrict__ w2,
    const bf16* __restrict__ w3, const bf16* __restrict__ cf, bf16* out, int8_t* tail, long long P, int use_norm,
    int residual) {
  using G = Geo<C, HIDDEN>;
  constexpr int HID = G::HID, KS = G::KS;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;

  const __amdgpu_buffer_rsrc_t r1 = buffer_rsrc(w1, HID * C * 2);
  const __amdgpu_buffer_rsrc_t r2 = buffer_rsrc(w2, HID * C * 2);
  const __amdgpu_buffer_rsrc_t r3 = buffer_rsrc(w3, C * HID * 2);
  const __amdgpu_buffer_rsrc_t rc = buffer_rsrc(cf, 2 * HID * 2 * 2);
  // The copies of a stage, each 1 KB into LDS chunk j of its tile: this wave
  // takes fc1 rows and fc2 rows j = wave + 4 q and fc3 columns j = wave + 4 q;
  // wave 0 also the bias pairs of both (4 bytes per lane).  The assignment is
  // fixed per wave, so a stage is straight-line code with a few offsets.
  static_assert(G::W12Copies % 4 == 0 && G::W3Copies % 4 == 0, "copies split evenly over the 4 waves");
  constexpr int Q12 = G::W12Copies / 4, Q3 = G::W3Copies / 4;
  unsigned vo12[Q12], vo3[Q3];
#pragma unroll
  for (int q = 0; q < Q12; ++q) {
    const int p = (wave + 4 * q) * 64 + lane, r = p / G::RowChunks, c = (p % G::RowChunks) ^ w12_swz<C>(r);
    vo12[q] = (unsigned)(r * C + c * 8) * 2;
  }
#pragma unroll
  for (int q = 0; q < Q3; ++q) {
    // LDS row 32 cb + m <- fc3 row 32 cb + 16 ((m & 15) >> 3) + 8 (m >> 4) + (m & 7)
    const int p = (wave + 4 * q) * 64 + lane, r = p >> 2, c = (p & 3) ^ swz4(r);
    const int m = r & 31, rg = (r & ~31) + 16 * ((m & 15) >> 3) + 8 * (m >> 4) + (m & 7);
    vo3[q] = (unsigned)(rg * HID + c * 8) * 2;
  }
  const unsigned vob = (unsigned)(((lane >> 5) * HID + (lane & 31)) * 2) * 2;
  auto stage_chunk = [&](int hc) {
    bf16* st = smem + (hc & 1) * G::Stage;
#pragma unroll
    for (int q = 0; q < Q12; ++q) {
      copy16_to_lds(r1, st + (wave + 4 * q) * 512, vo12[q], (unsigned)(hc * HC * C) * 2);
      copy16_to_lds(r2, st + G::W12Tile + (wave + 4 * q) * 512, vo12[q], (unsigned)(hc * HC * C) * 2);
    }
#pragma unroll
    for (int q = 0; q < Q3; ++q)
      copy16_to_lds(r3, st + 2 * G::W12Tile + (wave + 4 * q) * 512, vo3[q], (unsigned)(hc * HC) * 2);
    if (use_norm && wave == 0) copy4_to_lds(rc, st + 2 * G::W12Tile + G::W3Tile, vob, (unsigned)(hc * HC * 2) * 2);
  };

  stage_chunk(0);

  // This wave's 32 rows: lane (n, hh) holds chunks 2 s + hh of row p0 + n.
  const long long p0 = (long long)blockIdx.x * kRowsPerWg + wave * 32;
  const long long pair = p0 + n;
  const bool valid = pair < P;
  bf16x8 xf[KS];
  {
    float v[C / 2];
    const bf16* row = x + (size_t)(valid ? pair : 0) * C + 8 * hh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 raw;
      if (valid) {
        raw = load8(row + 16 * s);
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) raw[t] = f2bf(0.f);
      }
      unpack8(raw, v + 8 * s);
    }
    if (use_norm) {
      // affine-free LayerNorm over the C channels of lanes l and l ^ 32 (two-pass, fp32)
      float sum = 0.f;
#pragma unroll
      for (int c = 0; c < C / 2; ++c) sum += v[c];
      sum += __shfl_xor(sum, 32);
      const float mean = sum * (1.0f / C);
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < C / 2; ++c) {
        const float d = v[c] - mean;
        ss += d * d;
      }
      ss += __shfl_xor(ss, 32);
      const float rstd = valid ? rsqrtf(ss * (1.0f / C) + 1e-5f) : 0.f;
#pragma unroll
      for (int c = 0; c < C / 2; ++c) xf[c >> 3][c & 7] = f2bf((v[c] - mean) * rstd);
    } else {
#pragma unroll
      for (int c = 0; c < C / 2; ++c) xf[c >> 3][c & 7] = f2bf(v[c]);
    }
  }
  const bf16x8 xb = bias_step_x(valid, hh);
  const int rw = perm32(n);   // weight row read by this lane in the fc1 / fc2 blocks

  f32x16 acc[C / 32];
#pragma unroll
  for (int cb = 0; cb < C / 32; ++cb) acc[cb] = zero16();

#pragma unroll 1
  for (int hc = 0; hc < G::NCH; ++hc) {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of chunk hc landed
    __syncthreads();                       // ... and everyone's; the other stage is free again
    if (hc + 1 < G::NCH) stage_chunk(hc + 1);
    const bf16* st = smem + (hc & 1) * G::Stage;
    const bf16* s1 = st;
    const bf16* s2 = st + G::W12Tile;
    const bf16* s3 = st + 2 * G::W12Tile;
    const bf16* cl = st + 2 * G::W12Tile + G::W3Tile;
    // h^T blocks: lane (n = row slot, hh) holds hidden hc*32 + 16hh + u.
    f32x16 a = zero16(), g = zero16();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      a = mfma32(load8(s1 + w12_off<C>(rw, 2 * s + hh)), xf[s], a);
      g = mfma32(load8(s2 + w12_off<C>(rw, 2 * s + hh)), xf[s], g);
    }
    if (use_norm) {
      a = mfma32(bias_step_w(cl, rw, hh), xb, a);
      g = mfma32(bias_step_w(cl, HC + rw, hh), xb, g);
    }
    bf16x8 hb[2];
#pragma unroll
    for (int u = 0; u < 16; ++u) hb[u >> 3][u & 7] = f2bf(siluf_fast(a[u]) * g[u]);
#pragma unroll
    for (int cb = 0; cb < C / 32; ++cb) {
      const int r = cb * 32 + perm32(n);
      acc[cb] = mfma32(load8(s3 + w3_off(r, 2 * hh)), hb[0], acc[cb]);
      acc[cb] = mfma32(load8(s3 + w3_off(r, 2 * hh + 1)), hb[1], acc[cb]);
    }
  }

  // D lane (n, hh) of block cb, register u: output channel
  // 32 cb + 16 (u >> 3) + 8 hh + (u & 7) of row p0 + n.  The two lanes of a
  // row are valid together (the tail exchange pairs them).
  if (!valid) return;
#pragma unroll
  for (int cb = 0; cb < C / 32; ++cb) {
    const size_t off0 = (size_t)pair * C + cb * 32 + 8 * hh, off1 = off0 + 16;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = acc[cb][u];
    if (kTail) {
      float xv[16];
      const size_t toff = (size_t)pair * C + cb * 32 + 16 * hh;
      tail_decode16(load8(res + off0), load8(res + off1), exchange_tail_halves(load_tail16(tail + toff), hh), xv);
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] += xv[u];
      bf16x8 lo, hi;
      u32x4 tb;
      tail_encode16(v, lo, hi, tb);
      store8(out + off0, lo);
      store8(out + off1, hi);
      *reinterpret_cast<u32x4*>(tail + toff) = exchange_tail_halves(tb, hh);
      continue;
    }
    if (residual) {
      const bf16x8 q0 = load8(res + off0), q1 = load8(res + off1);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        v[u] += bf2f(q0[u]);
        v[8 + u] += bf2f(q1[u]);
      }
    }
    bf16x8 lo, hi;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      lo[u] = f2bf(v[u]);
      hi[u] = f2bf(v[8 + u]);
    }
    store8(out + off0, lo);
    store8(out + off1, hi);
  }
}

template <int C, int HIDDEN>
int launch_rows(const bf16* x, const bf16* res, const bf16* w1, const bf16* w2, const bf16* w3, const bf16* cf,
                bf16* out, int8_t* tail, long long P, int use_norm, int residual, hipStream_t stream) {
  auto* kern = tail ? transition_rows_kernel<C, HIDDEN, true> : transition_rows_kernel<C, HIDDEN, false>;
  constexpr int smem = Geo<C, HIDDEN>::Smem;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, smem) !=
      hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "transition_pair: cannot set dynamic LDS size");
  const long long nwg = (P + kRowsPerWg - 1) / kRowsPerWg;
  if (nwg > 0x7fffffffLL) return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: too many rows");
  KernelTimerScope timed(C == 128 ? "transition_pair" : "transition_msa", stream);
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(kThreads), smem, stream, x, res, w1, w2, w3, cf, out, tail, P,
                     use_norm, residual);
  return check_launch("transition_pair");
}

}  // namespace

static bool supported(int64_t Dc, int64_t hidden) {
  return (Dc == 64 || Dc == 128) && (hidden == 4 * Dc || hidden == 2 * Dc);
}

int transition_pair_res(const void* x, const void* res, const float* norm_w, const float* norm_b, const void* fc1_w,
                        const void* fc2_w, const void* fc3_w, void* out, int8_t* res_tail, void* workspace,
                        size_t workspace_bytes, int64_t P, int64_t Dc, int64_t hidden, int use_norm, int residual,
                        hipStream_t stream) {
  if (!supported(Dc, hidden))
    return set_error(BIOEMU_ERR_UNSUPPORTED,
                     "transition_pair: dim must be 64 or 128 with hidden 4*dim or 2*dim (got %lld, %lld)",
                     (long long)Dc, (long long)hidden);
  if (P <= 0) return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: bad row count %lld", (long long)P);
  if (res_tail && (!residual || !aligned16(res_tail)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: res_tail needs residual=1 and 16-byte alignment");
  if (!x || !fc1_w || !fc2_w || !fc3_w || !out || !workspace || (use_norm && (!norm_w || !norm_b)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(fc1_w) || !aligned16(fc2_w) || !aligned16(fc3_w) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: tensors must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: out may alias x only with residual=1");
  if (residual && (!res || !aligned16(res)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: the residual base must be a 16-byte aligned tensor");
  const size_t need = supported(Dc, hidden) ? fold_bytes(2 * hidden, Dc) : 0;
  if (workspace_bytes < need)
    return set_error(BIOEMU_ERR_WORKSPACE, "transition_pair: workspace %zu < required %zu", workspace_bytes, need);

  // Folded fc1 | fc2 (one [2 hidden][Dc] matrix) and their bias pairs ([2 hidden][2]).
  char* p = static_cast<char*>(workspace);
  bf16* wf = reinterpret_cast<bf16*>(p);
  bf16* cf = reinterpret_cast<bf16*>(p + round_up(2 * hidden * Dc * 2, 256));
  const bf16* w1 = static_cast<const bf16*>(fc1_w);
  const bf16* w2 = static_cast<const bf16*>(fc2_w);
  if (use_norm) {
    const int rc = launch_fold_ln2(fc1_w, fc2_w, hidden, norm_w, norm_b, wf, cf, 2 * hidden, stream, (int)Dc);
    if (rc) return rc;
    w1 = wf;
    w2 = wf + hidden * Dc;
  }
  const bf16* xb = static_cast<const bf16*>(x);
  const bf16* rb = static_cast<const bf16*>(res);
  const bf16* w3 = static_cast<const bf16*>(fc3_w);
  bf16* ob = static_cast<bf16*>(out);
  const long long rows = (long long)P;
  if (Dc == 128)
    return hidden == 512
               ? launch_rows<128, 512>(xb, rb, w1, w2, w3, cf, ob, res_tail, rows, use_norm, residual, stream)
               : launch_rows<128, 256>(xb, rb, w1, w2, w3, cf, ob, res_tail, rows, use_norm, residual, stream);
  return hidden == 256 ? launch_rows<64, 256>(xb, rb, w1, w2, w3, cf, ob, res_tail, rows, use_norm, residual, stream)
                       : launch_rows<64, 128>(xb, rb, w1, w2, w3, cf, ob, res_tail, rows, use_norm, residual, stream);
}

}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_transition_pair_workspace_bytes(int64_t Dc, int64_t hidden) {
  if (!supported(Dc, hidden)) return 0;
  return fold_bytes(2 * hidden, Dc);
}

extern "C" int bioemu_transition_pair_fwd(const void* x, const float* norm_w, const float* norm_b,
                                          const void* fc1_w, const void* fc2_w, const void* fc3_w,
                                          void* out, int8_t* res_tail, void* workspace, size_t workspace_bytes,
                                          int64_t P, int64_t Dc, int64_t hidden, int use_norm, int residual,
                                          hipStream_t stream) {
  return transition_pair_res(x, x, norm_w, norm_b, fc1_w, fc2_w, fc3_w, out, res_tail, workspace, workspace_bytes,
                             P, Dc, hidden, use_norm, residual, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the same kernels, with the folded-weight workspace
// in a static device array instead of a caller-provided buffer.
//
// The workspace of bioemu_transition_pair_fwd does not grow with the row count:
// it holds fc1 | fc2 with the LayerNorm folded in and their bias pairs, at most
// fold_bytes(2 * 512, 128) = 266240 bytes (D = 128, hidden = 512).  Every GPU
// the library runs on holds one copy of `scratch` until the process ends; its
// device address is looked up once per device (hipGetSymbolAddress) on the
// first call made with that device current.  Each call rewrites every byte it
// reads (the fold kernels write all folded rows before the row kernel runs), so
// nothing needs clearing between calls; calls that overlap on one GPU (other
// streams, other threads) share the array and race.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = 266240;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(BIOEMU_ERR_LAUNCH, "transition_pair_noalloc: no current device (or device id >= %d)",
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(BIOEMU_ERR_LAUNCH, "transition_pair_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return BIOEMU_OK;
}
}  // namespace

extern "C" int bioemu_transition_pair_fwd_noalloc(const void* x, const float* norm_w, const float* norm_b,
                                                  const void* fc1_w, const void* fc2_w, const void* fc3_w,
                                                  void* out, int8_t* res_tail, int64_t P, int64_t Dc,
                                                  int64_t hidden, int use_norm, int residual, hipStream_t stream) {
  const size_t need = bioemu_transition_pair_workspace_bytes(Dc, hidden);
  if (need > kScratchBytes)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "transition_pair_noalloc: dim %lld / hidden %lld need %zu bytes of scratch, "
                     "more than the static %zu", (long long)Dc, (long long)hidden, need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return bioemu_transition_pair_fwd(x, norm_w, norm_b, fc1_w, fc2_w, fc3_w, out, res_tail, ws, kScratchBytes, P, Dc,
                                    hidden, use_norm, residual, stream);
}
