// Pair Transition (SwiGLU MLP) for gfx950.
//
// Reference: Transition.forward (src/bioemu2/biomoa/ops/transition.py:52-91):
//   xn = LN(x) (eps 1e-5, with bias) when use_norm;  out = fc3(silu(fc1(xn)) * fc2(xn))
// with c = 128 and hidden = 4c = 512 for the pair representation, no biases.
//
// The LayerNorm affine is folded into fc1 / fc2 once per call (fold.hip):
//   LN(x) W^T = xhat (W diag(gamma))^T + W beta
// so a wave normalises its pair tile affine-free and adds W beta with one
// extra MFMA k-step (pairtile.h).
//
// One workgroup = 4 waves x 32 pairs.  Each wave keeps its normalised pair
// tile in registers as MFMA operands and its 32x128 output accumulator in
// registers; the hidden dimension is walked in chunks of 32.  A chunk's weight
// slices (fc1 and fc2 rows, the fc3 columns and the two bias columns, 24.25 KB)
// are copied by buffer loads straight into LDS (no registers), double-buffered:
// chunk h + 1 is in flight while chunk h is multiplied.  The hidden
// activations never leave registers: silu(a) * b comes out of the fc1 / fc2
// MFMAs in exactly the layout fc3 consumes as its B operand.
//
// LDS tiles are unpadded (the copies write 1 KB runs); the 16-byte chunk index
// of each row is XOR-swizzled so that the perm32 row pattern of the operand
// reads hits 16 distinct bank groups per 16 lanes.
#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int C = 128;
constexpr int HID = 512;
constexpr int HC = 32;                      // hidden chunk
constexpr int NCH = HID / HC;               // 16 chunks
constexpr int kThreads = 256;               // 4 waves
constexpr int kPairsPerWg = 128;
constexpr int kW12Tile = HC * C;            // bf16: [32 rows][16 chunks]
constexpr int kW3Tile = C * HC;             // bf16: [128 rows][4 chunks]
constexpr int kBiasElems = 2 * HC * 2;      // bf16: [fc1 | fc2][32 rows][hi, lo]
constexpr int kStage = 2 * kW12Tile + kW3Tile + kBiasElems;
constexpr int kSmem = 2 * kStage * 2;       // bytes
constexpr int kCopies = 3 * 8 + 1;          // 1 KB copies per stage (+ the 256-byte bias copy)

__device__ __forceinline__ int swz16(int r) { return (r & 7) | ((r & 16) >> 1); }
__device__ __forceinline__ int swz4(int r) { return ((r >> 2) & 1) | (((r >> 4) & 1) << 1); }
__device__ __forceinline__ int w12_off(int r, int c) { return (r * 16 + (c ^ swz16(r))) * 8; }
__device__ __forceinline__ int w3_off(int r, int c) { return (r * 4 + (c ^ swz4(r))) * 8; }

// 16 (or 4) bytes per lane from a buffer straight into LDS at lds + 16 (4) * lane.
__device__ __forceinline__ void copy16_to_lds(__amdgpu_buffer_rsrc_t r, const bf16* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void copy4_to_lds(__amdgpu_buffer_rsrc_t r, const bf16* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 4, voff, soff, 0, 0);
}

__global__ __launch_bounds__(kThreads) void transition_pair_kernel(
    const bf16* x, const bf16* __restrict__ w1, const bf16* __restrict__ w2, const bf16* __restrict__ w3,
    const bf16* __restrict__ cf, bf16* out, long long P, int use_norm, int residual) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;

  const __amdgpu_buffer_rsrc_t r1 = buffer_rsrc(w1, HID * C * 2);
  const __amdgpu_buffer_rsrc_t r2 = buffer_rsrc(w2, HID * C * 2);
  const __amdgpu_buffer_rsrc_t r3 = buffer_rsrc(w3, C * HID * 2);
  const __amdgpu_buffer_rsrc_t rc = buffer_rsrc(cf, 2 * HID * 2 * 2);
  // Copy k of a stage (k = wave, wave + 4, ...): 0-7 fc1 rows, 8-15 fc2 rows,
  // 16-23 fc3 columns (1 KB each, LDS chunk 64 j + lane of the tile), 24 the
  // bias pairs of both (4 bytes per lane).
  auto stage_chunk = [&](int hc) {
    bf16* st = smem + (hc & 1) * kStage;
#pragma unroll
    for (int k = wave; k < kCopies; k += 4) {
      if (k < 16) {
        const int j = k & 7, p = j * 64 + lane, r = p >> 4, c = (p & 15) ^ swz16(r);
        copy16_to_lds(k < 8 ? r1 : r2, st + (k < 8 ? 0 : kW12Tile) + j * 512, (unsigned)(r * C + c * 8) * 2,
                        (unsigned)(hc * HC * C) * 2);
      } else if (k < 24) {
        const int j = k - 16, p = j * 64 + lane, r = p >> 2, c = (p & 3) ^ swz4(r);
        copy16_to_lds(r3, st + 2 * kW12Tile + j * 512, (unsigned)(r * HID + c * 8) * 2, (unsigned)(hc * HC) * 2);
      } else if (use_norm) {
        const int which = lane >> 5, row = lane & 31;
        copy4_to_lds(rc, st + 2 * kW12Tile + kW3Tile, (unsigned)((which * HID + row) * 2) * 2,
                       (unsigned)(hc * HC * 2) * 2);
      }
    }
  };

  stage_chunk(0);

  // This wave's 32 pairs: lane (n, hh) holds channel half hh of pair p0 + n.
  const long long p0 = (long long)blockIdx.x * kPairsPerWg + wave * 32;
  const long long pair = p0 + n;
  const bool valid = pair < P;
  bf16x8 xf[8];
  {
    float v[64];
    load_half_row_f32(x + (size_t)(valid ? pair : 0) * C, hh, valid, v);
    if (use_norm) {
      normalize_half_row(v, valid, xf);
    } else {
#pragma unroll
      for (int c = 0; c < 64; ++c) xf[c >> 3][c & 7] = f2bf(v[c]);
    }
  }
  const bf16x8 xb = bias_step_x(valid, hh);
  const int rw = perm32(n);   // weight row read by this lane in the fc1 / fc2 blocks

  f32x16 acc[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) acc[cb] = zero16();

#pragma unroll 1
  for (int hc = 0; hc < NCH; ++hc) {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of chunk hc landed
    __syncthreads();                       // ... and everyone's; the other stage is free again
    if (hc + 1 < NCH) stage_chunk(hc + 1);
    const bf16* st = smem + (hc & 1) * kStage;
    const bf16* s1 = st;
    const bf16* s2 = st + kW12Tile;
    const bf16* s3 = st + 2 * kW12Tile;
    const bf16* cl = st + 2 * kW12Tile + kW3Tile;
    // h^T blocks: lane (n = pair slot, hh) holds hidden hc*32 + 16hh + u.
    f32x16 a = zero16(), g = zero16();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      a = mfma32(load8(s1 + w12_off(rw, 8 * hh + s)), xf[s], a);
      g = mfma32(load8(s2 + w12_off(rw, 8 * hh + s)), xf[s], g);
    }
    if (use_norm) {
      a = mfma32(bias_step_w(cl, rw, hh), xb, a);
      g = mfma32(bias_step_w(cl, HC + rw, hh), xb, g);
    }
    bf16x8 hb[2];
#pragma unroll
    for (int u = 0; u < 16; ++u) hb[u >> 3][u & 7] = f2bf(siluf_fast(a[u]) * g[u]);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const int r = cb * 32 + perm32(n);
      acc[cb] = mfma32(load8(s3 + w3_off(r, 2 * hh)), hb[0], acc[cb]);
      acc[cb] = mfma32(load8(s3 + w3_off(r, 2 * hh + 1)), hb[1], acc[cb]);
    }
  }

  // D lane (n, hh) of block cb: output channel cb*32 + 16hh + u of pair p0 + n
  if (!valid) return;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const size_t off = (size_t)pair * C + cb * 32 + 16 * hh;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = acc[cb][u];
    if (residual) {
      const bf16x8 q0 = load8(x + off), q1 = load8(x + off + 8);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        v[u] += bf2f(q0[u]);
        v[8 + u] += bf2f(q1[u]);
      }
    }
    store16(out + off, v);
  }
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" size_t bioemu_transition_pair_workspace_bytes(int64_t Dc, int64_t hidden) {
  if (Dc != C || hidden != HID) return 0;
  return fold_bytes(2 * HID);
}

extern "C" int bioemu_transition_pair_fwd(const void* x, const float* norm_w, const float* norm_b,
                                          const void* fc1_w, const void* fc2_w, const void* fc3_w,
                                          void* out, void* workspace, size_t workspace_bytes, int64_t P,
                                          int64_t Dc, int64_t hidden, int use_norm, int residual,
                                          hipStream_t stream) {
  if (Dc != C || hidden != HID)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "transition_pair: only dim=128, hidden=512 supported (got %lld, %lld)",
                     (long long)Dc, (long long)hidden);
  if (P <= 0) return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: bad row count %lld", (long long)P);
  if (!x || !fc1_w || !fc2_w || !fc3_w || !out || !workspace || (use_norm && (!norm_w || !norm_b)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(fc1_w) || !aligned16(fc2_w) || !aligned16(fc3_w) ||
      !aligned16(workspace))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: tensors must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: out may alias x only with residual=1");
  const size_t need = bioemu_transition_pair_workspace_bytes(Dc, hidden);
  if (workspace_bytes < need)
    return set_error(BIOEMU_ERR_WORKSPACE, "transition_pair: workspace %zu < required %zu", workspace_bytes, need);

  // Folded fc1 | fc2 (one [1024][128] matrix) and their bias pairs ([1024][2]).
  char* p = static_cast<char*>(workspace);
  bf16* wf = reinterpret_cast<bf16*>(p);
  bf16* cf = reinterpret_cast<bf16*>(p + round_up((int64_t)2 * HID * C * 2, 256));
  const bf16* w1 = static_cast<const bf16*>(fc1_w);
  const bf16* w2 = static_cast<const bf16*>(fc2_w);
  if (use_norm) {
    int rc = launch_fold_ln(fc1_w, norm_w, norm_b, wf, cf, HID, stream);
    if (!rc) rc = launch_fold_ln(fc2_w, norm_w, norm_b, wf + HID * C, cf + HID * 2, HID, stream);
    if (rc) return rc;
    w1 = wf;
    w2 = wf + HID * C;
  }
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(transition_pair_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "transition_pair: cannot set dynamic LDS size");
  const long long nwg = (P + kPairsPerWg - 1) / kPairsPerWg;
  if (nwg > 0x7fffffffLL) return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: too many rows");
  KernelTimerScope timed("transition_pair", stream);
  hipLaunchKernelGGL(transition_pair_kernel, dim3((unsigned)nwg), dim3(kThreads), kSmem, stream,
                     static_cast<const bf16*>(x), w1, w2, static_cast<const bf16*>(fc3_w), cf,
                     static_cast<bf16*>(out), (long long)P, use_norm, residual);
  return check_launch("transition_pair");
}
