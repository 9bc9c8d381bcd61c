// LayerNorm-into-projection folding (see pairtile.h):
//   W' = W diag(gamma)  (bf16),   c = W beta  (fp32, stored as bf16 hi + lo).
#include "common.h"
#include "internal.h"

namespace bioemu {
namespace {

// One wave per folded row, four rows per workgroup: lane l holds the kC / 64
// consecutive elements l * kC / 64 ..; W beta is a wave reduction.  Rows at or
// past rows1 come from the second matrix w2 (row r - rows1), so two
// projections that share the LayerNorm fold in one launch.
template <int kC>
__global__ __launch_bounds__(256) void fold_ln_kernel(const bf16* __restrict__ w, const bf16* __restrict__ w2,
                                                      int rows1, int rows, const float* __restrict__ gamma,
                                                      const float* __restrict__ beta, bf16* __restrict__ wf,
                                                      bf16* __restrict__ cf) {
  constexpr int E = kC / 64;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const bf16* src = r < rows1 ? w + (size_t)r * kC : w2 + (size_t)(r - rows1) * kC;
  float part = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = lane * E + e;
    const float wv = bf2f(src[c]);
    wf[(size_t)r * kC + c] = f2bf(wv * gamma[c]);
    if (beta) part += wv * beta[c];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) {
    const bf16 hi = f2bf(part);
    cf[2 * r] = hi;
    cf[2 * r + 1] = f2bf(part - bf2f(hi));
  }
}

}  // namespace

int launch_fold_ln2(const void* w, const void* w2, int64_t rows1, const float* gamma, const float* beta, void* wf,
                    void* cf, int64_t rows, hipStream_t stream, int width) {
  if (rows <= 0 || rows > 65535 || rows1 <= 0 || rows1 > rows)
    return set_error(BIOEMU_ERR_INVALID_ARG, "fold_ln: bad row count %lld (%lld from the first matrix)",
                     (long long)rows, (long long)rows1);
  if (width != 64 && width != 128 && width != 256)
    return set_error(BIOEMU_ERR_INVALID_ARG, "fold_ln: width %d unsupported", width);
  KernelTimerScope timed("fold_ln", stream);
  const dim3 grid((unsigned)((rows + 3) / 4));
  const bf16* a = static_cast<const bf16*>(w);
  const bf16* b = static_cast<const bf16*>(w2);
  bf16* o = static_cast<bf16*>(wf);
  bf16* c = static_cast<bf16*>(cf);
  if (width == 256)
    hipLaunchKernelGGL(fold_ln_kernel<256>, grid, dim3(256), 0, stream, a, b, (int)rows1, (int)rows, gamma, beta, o, c);
  else if (width == 128)
    hipLaunchKernelGGL(fold_ln_kernel<128>, grid, dim3(256), 0, stream, a, b, (int)rows1, (int)rows, gamma, beta, o, c);
  else
    hipLaunchKernelGGL(fold_ln_kernel<64>, grid, dim3(256), 0, stream, a, b, (int)rows1, (int)rows, gamma, beta, o, c);
  return check_launch("fold_ln");
}

int launch_fold_ln(const void* w, const float* gamma, const float* beta, void* wf, void* cf, int64_t rows,
                   hipStream_t stream, int width) {
  return launch_fold_ln2(w, w, rows, gamma, beta, wf, cf, rows, stream, width);
}

}  // namespace bioemu
