// Pair Transition (SwiGLU MLP) for gfx950.
//
// Reference: Transition.forward (src/bioemu2/biomoa/ops/transition.py:52-91):
//   xn = LN(x) (eps 1e-5, with bias) when use_norm;  out = fc3(silu(fc1(xn)) * fc2(xn))
// with c = 128 and hidden = 4c = 512 for the pair representation, no biases.
//
// One workgroup = 8 waves x 32 pairs.  Each wave keeps its LayerNorm'd pair
// tile in registers as MFMA operands and its 32x128 output accumulator in
// registers; the hidden dimension is walked in chunks of 32 whose fc1/fc2/fc3
// weight slices are staged in LDS (double-buffered) and shared by all waves.
// The hidden activations never leave registers: the SwiGLU product comes out
// of the fc1/fc2 MFMAs in exactly the layout fc3 consumes as its B operand.
#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int C = 128;
constexpr int HID = 512;
constexpr int HC = 32;                 // hidden chunk
constexpr int kThreads = 512;          // 8 waves
constexpr int kPairsPerWg = 256;
constexpr int LDW3 = HC + 8;           // LDS row stride (bf16) of the fc3 slice
constexpr int kStageElems = 2 * HC * kLdw + C * LDW3;
constexpr int kSmem = 2 * kStageElems * 2;

__device__ __forceinline__ void stage_chunk(bf16* st, const bf16* __restrict__ w1, const bf16* __restrict__ w2,
                                            const bf16* __restrict__ w3, int hc) {
  bf16* s1 = st;
  bf16* s2 = st + HC * kLdw;
  bf16* s3 = st + 2 * HC * kLdw;
  // fc1 / fc2 rows hc*32 .. +31 (16 chunks of 8 each) = 1024 chunks; fc3 [128][32] = 512 chunks
  for (int q = threadIdx.x; q < 2 * HC * 16 + C * 4; q += blockDim.x) {
    if (q < 2 * HC * 16) {
      const int which = q / (HC * 16), r = (q / 16) % HC, part = q & 15;
      const bf16* src = (which ? w2 : w1) + (size_t)(hc * HC + r) * C + part * 8;
      store8((which ? s2 : s1) + r * kLdw + part * 8, load8(src));
    } else {
      const int q3 = q - 2 * HC * 16;
      const int r = q3 >> 2, part = q3 & 3;
      store8(s3 + r * LDW3 + part * 8, load8(w3 + (size_t)r * HID + hc * HC + part * 8));
    }
  }
}

__global__ __launch_bounds__(kThreads) void transition_pair_kernel(
    const bf16* x, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    const bf16* __restrict__ w1, const bf16* __restrict__ w2, const bf16* __restrict__ w3, bf16* out,
    long long P, int use_norm, int residual) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* stage = reinterpret_cast<bf16*>(smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const long long pair = (long long)blockIdx.x * kPairsPerWg + wave * 32 + n;
  const bool valid = pair < P;

  stage_chunk(stage, w1, w2, w3, 0);

  bf16x8 raw[8], xf[8];
  load_half_row(x + (size_t)(valid ? pair : 0) * C, hh, valid, raw);
  if (use_norm) {
    layernorm_half_row(raw, ln_w, ln_b, hh, 1e-5f, xf);
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) xf[s] = raw[s];
  }

  f32x16 acc[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) acc[cb] = zero16();

  for (int hc = 0; hc < HID / HC; ++hc) {
    __syncthreads();  // chunk hc staged; chunk hc-1's buffer free
    if (hc + 1 < HID / HC) stage_chunk(stage + ((hc + 1) & 1) * kStageElems, w1, w2, w3, hc + 1);
    const bf16* st = stage + (hc & 1) * kStageElems;
    // h^T block: lane (n = pair, hh) holds hidden 16hh + u of this chunk.
    const f32x16 a = proj_block_pm(xf, st, 0, n, hh);
    const f32x16 g = proj_block_pm(xf, st + HC * kLdw, 0, n, hh);
    bf16x8 hb[2];
#pragma unroll
    for (int u = 0; u < 16; ++u) hb[u >> 3][u & 7] = f2bf(siluf_fast(a[u]) * g[u]);
    const bf16* s3 = st + 2 * HC * kLdw;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const bf16* wr = s3 + (cb * 32 + perm32(n)) * LDW3 + 16 * hh;
      acc[cb] = mfma32(load8(wr), hb[0], acc[cb]);
      acc[cb] = mfma32(load8(wr + 8), hb[1], acc[cb]);
    }
  }

  if (!valid) return;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const size_t off = (size_t)pair * C + cb * 32 + 16 * hh;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = acc[cb][u];
    if (residual) {
      const bf16x8 r0 = load8(x + off), r1 = load8(x + off + 8);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        v[u] += bf2f(r0[u]);
        v[8 + u] += bf2f(r1[u]);
      }
    }
    store16(out + off, v);
  }
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" int bioemu_transition_pair_fwd(const void* x, const float* norm_w, const float* norm_b,
                                          const void* fc1_w, const void* fc2_w, const void* fc3_w,
                                          void* out, int64_t P, int64_t Dc, int64_t hidden,
                                          int use_norm, int residual, hipStream_t stream) {
  if (Dc != C || hidden != HID)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "transition_pair: only dim=128, hidden=512 supported (got %lld, %lld)",
                     (long long)Dc, (long long)hidden);
  if (P <= 0) return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: bad row count %lld", (long long)P);
  if (!x || !fc1_w || !fc2_w || !fc3_w || !out || (use_norm && (!norm_w || !norm_b)))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: null pointer argument");
  if (!aligned16(x) || !aligned16(out) || !aligned16(fc1_w) || !aligned16(fc2_w) || !aligned16(fc3_w))
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: tensors must be 16-byte aligned");
  if (out == x && !residual)
    return set_error(BIOEMU_ERR_INVALID_ARG, "transition_pair: out may alias x only with residual=1");
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(transition_pair_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kSmem) != hipSuccess)
    return set_error(BIOEMU_ERR_LAUNCH, "transition_pair: cannot set dynamic LDS size");
  const long long nwg = (P + kPairsPerWg - 1) / kPairsPerWg;
  KernelTimerScope timed("transition_pair", stream);
  hipLaunchKernelGGL(transition_pair_kernel, dim3((unsigned)nwg), dim3(kThreads), kSmem, stream,
                     static_cast<const bf16*>(x), norm_w, norm_b, static_cast<const bf16*>(fc1_w),
                     static_cast<const bf16*>(fc2_w), static_cast<const bf16*>(fc3_w),
                     static_cast<bf16*>(out), (long long)P, use_norm, residual);
  return check_launch("transition_pair");
}
