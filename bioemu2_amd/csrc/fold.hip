// LayerNorm-into-projection folding (see pairtile.h):
//   W' = W diag(gamma)  (bf16),   c = W beta  (fp32, stored as bf16 hi + lo).
#include "common.h"
#include "internal.h"

namespace bioemu {
namespace {

template <int kC>
__global__ __launch_bounds__(kC) void fold_ln_kernel(const bf16* __restrict__ w, const float* __restrict__ gamma,
                                                     const float* __restrict__ beta, bf16* __restrict__ wf,
                                                     bf16* __restrict__ cf) {
  __shared__ float red[kC];
  const int r = blockIdx.x, c = threadIdx.x;
  const float wv = bf2f(w[(size_t)r * kC + c]);
  wf[(size_t)r * kC + c] = f2bf(wv * gamma[c]);
  red[c] = beta ? wv * beta[c] : 0.f;
  __syncthreads();
  for (int st = kC / 2; st > 0; st >>= 1) {
    if (c < st) red[c] += red[c + st];
    __syncthreads();
  }
  if (c == 0) {
    const float tot = red[0];
    const bf16 hi = f2bf(tot);
    cf[2 * r] = hi;
    cf[2 * r + 1] = f2bf(tot - bf2f(hi));
  }
}

}  // namespace

int launch_fold_ln(const void* w, const float* gamma, const float* beta, void* wf, void* cf, int64_t rows,
                   hipStream_t stream, int width) {
  if (rows <= 0 || rows > 65535) return set_error(BIOEMU_ERR_INVALID_ARG, "fold_ln: bad row count %lld", (long long)rows);
  if (width != 64 && width != 128 && width != 256)
    return set_error(BIOEMU_ERR_INVALID_ARG, "fold_ln: width %d unsupported", width);
  KernelTimerScope timed("fold_ln", stream);
  if (width == 256)
    hipLaunchKernelGGL(fold_ln_kernel<256>, dim3((unsigned)rows), dim3(256), 0, stream, static_cast<const bf16*>(w),
                       gamma, beta, static_cast<bf16*>(wf), static_cast<bf16*>(cf));
  else if (width == 128)
    hipLaunchKernelGGL(fold_ln_kernel<128>, dim3((unsigned)rows), dim3(128), 0, stream, static_cast<const bf16*>(w),
                       gamma, beta, static_cast<bf16*>(wf), static_cast<bf16*>(cf));
  else
    hipLaunchKernelGGL(fold_ln_kernel<64>, dim3((unsigned)rows), dim3(64), 0, stream, static_cast<const bf16*>(w),
                       gamma, beta, static_cast<bf16*>(wf), static_cast<bf16*>(cf));
  return check_launch("fold_ln");
}

}  // namespace bioemu
