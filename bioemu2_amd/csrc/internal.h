// Host-side internals shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/bioemu2_mi355x.h"

namespace bioemu {

// Records a formatted message for bioemu_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// Checks the launch status of the most recent kernel launch.
int check_launch(const char* what);

// Brackets one kernel launch with hipEvents on `stream` while the kernel
// timer is enabled (bioemu_timer_enable); a no-op otherwise.
class KernelTimerScope {
 public:
  KernelTimerScope(const char* name, hipStream_t stream);
  ~KernelTimerScope();
  KernelTimerScope(const KernelTimerScope&) = delete;
  KernelTimerScope& operator=(const KernelTimerScope&) = delete;

 private:
  hipStream_t stream_;
  int name_idx_ = -1;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
};

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Batched bf16 "NT" GEMM: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k] for
// z < batch, with M = N = K = n (a multiple of kGemmTile) and bf16 output.
constexpr int kGemmTile = 128;
int launch_bgemm_nt(const void* A, const void* B, void* C, int64_t batch, int64_t n,
                    hipStream_t stream);

}  // namespace bioemu
