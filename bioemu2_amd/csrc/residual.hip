// Residual streams with int8 tails (common.h): conversion between an fp32
// tensor and its (bf16 value, int8 tail) pair, for callers that hand the
// block fp32 activations or want fp32 back.
//
// The reference's bf16-mixed trunk keeps z and s in bf16 and rounds them after
// every residual add (z = z + op(z) on bf16 tensors under autocast,
// src/bioemu2/biomoa/modules/pairmixer.py:446-456, model.py:216-223); carrying
// a tail keeps the residual stream at ~16 significant bits instead, so a stack
// of ops rounds once (when the stream is joined) rather than once per op.
#include "common.h"
#include "internal.h"

namespace bioemu {
namespace {

constexpr int kThreads = 256;

// One thread per 16 elements (n % 16 == 0, 16-byte aligned buffers).
__global__ __launch_bounds__(kThreads) void stream_split_kernel(const float* __restrict__ x, bf16* __restrict__ hi,
                                                                int8_t* __restrict__ tail, long long chunks) {
  const long long c = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (c >= chunks) return;
  float v[16];
  const f32x4* src = reinterpret_cast<const f32x4*>(x + 16 * c);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 t = src[q];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[4 * q + u] = t[u];
  }
  tail_store16(hi + 16 * c, tail + 16 * c, v);
}

__global__ __launch_bounds__(kThreads) void stream_join_kernel(const bf16* __restrict__ hi,
                                                               const int8_t* __restrict__ tail,
                                                               float* __restrict__ out, long long chunks) {
  const long long c = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (c >= chunks) return;
  float v[16];
  tail_decode16(load8(hi + 16 * c), load8(hi + 16 * c + 8), load_tail16(tail + 16 * c), v);
  f32x4* dst = reinterpret_cast<f32x4*>(out + 16 * c);
#pragma unroll
  for (int q = 0; q < 4; ++q) dst[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
}

int check_stream_args(const void* a, const void* b, const void* c, int64_t n, const char* what) {
  if (!a || !b || !c) return set_error(BIOEMU_ERR_INVALID_ARG, "%s: null pointer argument", what);
  if (n <= 0 || n % 16) return set_error(BIOEMU_ERR_INVALID_ARG, "%s: element count %lld must be a positive multiple of 16",
                                        what, (long long)n);
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return set_error(BIOEMU_ERR_INVALID_ARG, "%s: buffers must be 16-byte aligned", what);
  if (n / 16 / kThreads >= 0x7fffffffLL) return set_error(BIOEMU_ERR_INVALID_ARG, "%s: too many elements", what);
  return BIOEMU_OK;
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

extern "C" int bioemu_stream_split(const float* x, void* hi, int8_t* tail, int64_t n, hipStream_t stream) {
  int rc = check_stream_args(x, hi, tail, n, "stream_split");
  if (rc) return rc;
  const long long chunks = n / 16;
  KernelTimerScope timed("stream_split", stream);
  hipLaunchKernelGGL(stream_split_kernel, dim3((unsigned)((chunks + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     stream, x, static_cast<bf16*>(hi), tail, chunks);
  return check_launch("stream_split");
}

extern "C" int bioemu_stream_join(const void* hi, const int8_t* tail, float* out, int64_t n, hipStream_t stream) {
  int rc = check_stream_args(hi, tail, out, n, "stream_join");
  if (rc) return rc;
  const long long chunks = n / 16;
  KernelTimerScope timed("stream_join", stream);
  hipLaunchKernelGGL(stream_join_kernel, dim3((unsigned)((chunks + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     stream, static_cast<const bf16*>(hi), tail, out, chunks);
  return check_launch("stream_join");
}
