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

// Grid-stride pair-tile loops index their tiles in 32-bit unsigned arithmetic;
// launchers reject a tile count of 2^31 or more (far beyond any pair tensor
// that fits in device memory).
constexpr int64_t kMaxTiles = int64_t(1) << 31;

// Waves per workgroup for a persistent grid of one workgroup per CU that
// walks `tiles` equal tiles: more waves hide more latency (gain[c] = measured
// throughput of waves[c] relative to waves[0] when the tiles divide evenly),
// but a partial last round of tiles costs a whole round, so the pick
// minimises rounds x waves / gain.
inline int pick_waves_per_wg(int64_t tiles, int cus, const int* waves, const double* gain, int n) {
  int best = waves[0];
  double best_cost = 0;
  for (int c = 0; c < n; ++c) {
    const int64_t per_round = (int64_t)cus * waves[c];
    const double cost = (double)((tiles + per_round - 1) / per_round) * waves[c] / gain[c];
    if (c == 0 || cost < best_cost) {
      best = waves[c];
      best_cost = cost;
    }
  }
  return best;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Batched bf16 "NT" GEMM: C[z][i][j] = sum_k A[z][i][k] * B[z][j][k] for
// z < batch, with M = N = K = n (a multiple of kGemmTile) and bf16 output.
constexpr int kGemmTile = 256;
int launch_bgemm_nt(const void* A, const void* B, void* C, int64_t batch, int64_t n,
                    hipStream_t stream);

// LayerNorm folding (fold.hip): wf = W diag(gamma) [rows][width] bf16, cf = W beta
// as bf16 (hi, lo) pairs [rows][2]; beta may be null.  W is [rows][width] bf16,
// width 128 (default), 64 or 256.
int launch_fold_ln(const void* w, const float* gamma, const float* beta, void* wf, void* cf, int64_t rows,
                   hipStream_t stream, int width = 128);
// The same for two matrices that share gamma and beta, in one launch: rows
// [0, rows1) of the output fold w, rows [rows1, rows) fold w2 (its row r - rows1).
int launch_fold_ln2(const void* w, const void* w2, int64_t rows1, const float* gamma, const float* beta, void* wf,
                    void* cf, int64_t rows, hipStream_t stream, int width = 128);
inline size_t fold_bytes(int64_t rows, int64_t width = 128) {
  return (size_t)round_up(rows * width * 2, 256) + (size_t)round_up(rows * 4, 256);
}

// Token-side helpers (token.hip).  Rows are B batches of N tokens stored
// padded to Np rows each; see token.hip for the row conventions.
int token_layernorm(const void* x, const float* gamma, const float* beta, void* y, int64_t B, int64_t N,
                    int64_t Np, int64_t K, hipStream_t stream);
int token_gemm(int epi, bool trans, const void* A, const void* W, const void* W2, const float* col_bias,
               const void* res, void* out, int64_t M, int64_t K, int64_t Nout, int64_t N, int64_t Np,
               int64_t out_rows, hipStream_t stream, const char* name, int8_t* tail = nullptr);
constexpr int kEpiStoreId = 0, kEpiSigmoidId = 1, kEpiSwiGLUId = 2, kEpiResidualId = 3;
// q | k | v^T | g = sn [Wq; Wk; Wv; Wg]^T in one launch (w_qkv [3 c_s][c_s], w_g
// [c_s][c_s]): q = (. + q_bias) * q_scale, g = sigmoid(.), v written
// transposed per sequence of seq_rows rows; c_s % 64 == 0, M % seq_rows == 0.
// out = A W^T (+ res, with an optional int8 tail) on LDS-staged 256 x 256 tiles;
// rows and out_rows as token_gemm; K % 64 == 0, Nout % 32 == 0.
int token_out_proj(const void* A, const void* W, const void* res, void* out, int8_t* tail, int64_t M, int64_t K,
                   int64_t Nout, int64_t Np, int64_t out_rows, bool residual, hipStream_t stream, const char* name);
int token_qkvg(const void* sn, const void* wqkv, const void* w_g, const float* q_bias, float q_scale, void* q,
               void* k, void* vt, void* g, int64_t M, int64_t CS, int64_t seq_rows, hipStream_t stream,
               const char* name);

// Row transition out = res + fc3(silu(fc1 LN x) * fc2 LN x) (transition.hip): the
// arguments of bioemu_transition_pair_fwd plus the residual base res (x for
// the in-place block update; with res_tail, res is its hi part and out_tail
// = res_tail is rewritten in place).
int transition_pair_res(const void* x, const void* res, const float* norm_w, const float* norm_b, const void* fc1_w,
                        const void* fc2_w, const void* fc3_w, void* out, int8_t* res_tail, void* workspace,
                        size_t workspace_bytes, int64_t P, int64_t Dc, int64_t hidden, int use_norm, int residual,
                        hipStream_t stream);

}  // namespace bioemu
