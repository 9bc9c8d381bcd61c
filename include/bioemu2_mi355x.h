/*
 * bioemu2_mi355x — C ABI of the MI355X (gfx950) Pairformer hot-path kernels.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, runs
 * asynchronously on that stream, allocates nothing, and returns 0 or a
 * negative BIOEMU_ERR_* code (bioemu_last_error() gives the message).
 *
 * Data types:
 *   activations  bf16, channel-last ([B, N, N, C] pair tensors, [B, N, C] singles)
 *   masks        uint8 0/1
 *   LayerNorm    gamma/beta fp32
 *   Linear       weights bf16, row-major [out, in] (torch nn.Linear layout)
 * Arithmetic: bf16 MFMA operands with fp32 accumulation; LayerNorm statistics,
 * softmax and gates in fp32.  The *_f32 entry points (end of this file) take
 * fp32 activations and weights and compute in fp32 throughout.
 *
 * Scratch memory is caller-owned: each op with intermediates has a
 * *_workspace_bytes() query and takes (workspace, workspace_bytes).
 *
 * Residual tails.  Every entry point that can add its result into a residual
 * stream (residual=1, or z_res for the OPM) takes an optional `res_tail`: an
 * int8 plane with one byte per element of `out`.  The stream's value is then
 * hi + t * 2^(E(hi) - 142) (hi the bf16 element, E its biased exponent field,
 * t the tail byte: 1/256ths of hi's unit in the last place), ~16 significant
 * bits.  The op reads x + tail, adds its update in fp32 and writes the sum
 * back as a bf16 element plus a new tail byte (the tail is updated in place).
 * Inputs that an op only normalises are read as bf16 (the tail is not read).
 * res_tail = NULL keeps the plain bf16 stream, rounded after every add (the
 * reference's bf16-autocast trunk).  bioemu_stream_split / _join convert
 * between fp32 tensors and (bf16, tail) pairs.
 */
#ifndef BIOEMU2_MI355X_H
#define BIOEMU2_MI355X_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BIOEMU_OK 0
#define BIOEMU_ERR_INVALID_ARG (-1)
#define BIOEMU_ERR_UNSUPPORTED (-2)
#define BIOEMU_ERR_WORKSPACE (-3)
#define BIOEMU_ERR_LAUNCH (-4)

/* Library version string and the message of the last failing call (per thread). */
const char* bioemu_version(void);
const char* bioemu_last_error(void);

/*
 * Kernel timer (instrumentation; no counterpart in the reference, which times
 * whole calls with CUDA events, examples/search_batch_size.py:28-46).
 * While enabled, every kernel this library launches is bracketed by two
 * hipEvents on its launch stream.  bioemu_timer_query() synchronises on the
 * pending events and returns, per kernel name, the launch count and the summed
 * event-to-event duration in milliseconds.
 */
int bioemu_timer_enable(int on);
int bioemu_timer_reset(void);
int bioemu_timer_count(void);
int bioemu_timer_query(int idx, char* name, size_t name_len, int64_t* launches, double* total_ms);

/*
 * Triangle multiplicative update, outgoing (outgoing=1) or incoming (0).
 *
 * Replaces TriangleMultiplicationFull.forward / TriangleMultiplicationCueq.forward
 * (src/bioemu2/biomoa/ops/triangle_multiplication.py:89-99 and :137-151):
 *   xn  = LN_in(x);  p = p_in(xn) * sigmoid(g_in(xn));  p[~mask] = 0
 *   a, b = p[..., :D], p[..., D:]
 *   o[i,j] = sum_k a[i,k] * b[j,k]       (outgoing)
 *   o[i,j] = sum_k a[k,i] * b[k,j]       (incoming)
 *   out = p_out(LN_out(o)) * sigmoid(g_out(xn))   (+ x when residual != 0)
 * x, out: [B,N,N,D] bf16 (out may equal x when residual != 0); mask [B,N,N].
 * p_in_w, g_in_w: [2D, D]; p_out_w, g_out_w: [D, D].  D must be 128; N <= 9472.
 * res_tail: NULL or the [B,N,N,D] int8 tail of the residual stream (residual=1).
 */
size_t bioemu_trimul_workspace_bytes(int64_t B, int64_t N, int64_t D);
int bioemu_trimul_fwd(const void* x, const uint8_t* mask, const float* norm_in_w,
                      const float* norm_in_b, const void* p_in_w, const void* g_in_w,
                      const float* norm_out_w, const float* norm_out_b, const void* p_out_w,
                      const void* g_out_w, void* out, int8_t* res_tail, void* workspace,
                      size_t workspace_bytes,
                      int64_t B, int64_t N, int64_t D, int outgoing, int residual,
                      hipStream_t stream);

/*
 * Triangle attention around the starting node (starting=1) or ending node (0).
 *
 * No counterpart in the reference (biomoa/modules/pairmixer.py:459-462 removed
 * it); AlphaFold3 suppl. Alg. 14/15 with the reference's attention masking
 * convention (masked keys replaced by -1e6, attention_pair_bias.py:184-190).
 * It would bind through the make() 3-tuple registry form
 * (src/bioemu2/biomoa/utils/strategy.py:33-36).  Per batch, frame row i, head h
 * (frame = z for starting, z^T for ending):
 *   zn = LN(z); q,k,v,g,bias = zn W^T (g through a sigmoid; bias has H columns)
 *   o[i,j] = sum_k softmax_k(q[i,j].k[i,k]/sqrt(d) + bias[j,k,h]; mask[i,k]) v[i,k]
 *   update[i,j] = (g[i,j] * o[i,j]) Wo^T    (+ z when residual != 0)
 * z, out: [B,N,N,D] bf16 (out may equal z when residual != 0); mask [B,N,N].
 * w_proj: [4*D + H, D] = rows of Wq, Wk, Wv, Wg, Wbias; w_o: [D, D].
 * D must be 128 and H 4 (head dim 32).
 * res_tail: NULL or the [B,N,N,D] int8 tail of the residual stream (residual=1).
 */
size_t bioemu_triatt_workspace_bytes(int64_t B, int64_t N, int64_t D, int64_t H);
int bioemu_triatt_fwd(const void* z, const uint8_t* mask, const float* norm_w, const float* norm_b,
                      const void* w_proj, const void* w_o, void* out, int8_t* res_tail, void* workspace,
                      size_t workspace_bytes, int64_t B, int64_t N, int64_t D, int64_t H,
                      int starting, int residual, hipStream_t stream);

/*
 * Row Transition (SwiGLU MLP), fused: LN -> fc1/fc2 -> silu(a)*b -> fc3 (+ x).
 * Replaces Transition.forward (src/bioemu2/biomoa/ops/transition.py:52-91) for
 * the pair representation (D 128, hidden 512) and the MSA representation
 * (D 64, hidden 256; biomoa/modules/pairmixer.py:631-634).  x, out: [P, D] bf16
 * rows (P = B*N*N pairs or B*S*N MSA entries), out may equal x when
 * residual != 0.  fc1_w, fc2_w: [hidden, D]; fc3_w: [D, hidden].  D must be 128
 * or 64 and hidden 4*D or 2*D (the denoiser's PairwiseConditioning transitions,
 * diffusion.py:498-507).  use_norm=0 skips the LayerNorm (norm_* unused).
 * The workspace holds fc1/fc2 with the LayerNorm affine folded in (size from
 * bioemu_transition_pair_workspace_bytes, independent of P).
 * res_tail: NULL or the [P, D] int8 tail of the residual stream (residual=1).
 */
size_t bioemu_transition_pair_workspace_bytes(int64_t D, int64_t hidden);
int bioemu_transition_pair_fwd(const void* x, const float* norm_w, const float* norm_b,
                               const void* fc1_w, const void* fc2_w, const void* fc3_w, void* out,
                               int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t P, int64_t D,
                               int64_t hidden, int use_norm, int residual, hipStream_t stream);

/*
 * Allocation-free variant of bioemu_transition_pair_fwd (same arguments minus
 * the workspace, same kernels, bit-identical results).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * The folded-weight scratch (at most 266240 bytes: D = 128, hidden = 512) lives
 * in a static device array, one per GPU, held until the process ends; its
 * address is looked up once per device on the first call with that device
 * current.  Every call on one GPU shares that array: calls that overlap on a
 * GPU (other streams or threads) race.  Each call rewrites all the scratch it
 * reads, so nothing needs clearing between calls.  Rejects shapes whose scratch
 * would exceed the array (BIOEMU_ERR_UNSUPPORTED).
 */
int bioemu_transition_pair_fwd_noalloc(const void* x, const float* norm_w, const float* norm_b,
                                       const void* fc1_w, const void* fc2_w, const void* fc3_w, void* out,
                                       int8_t* res_tail, int64_t P, int64_t D, int64_t hidden, int use_norm,
                                       int residual, hipStream_t stream);

/*
 * Token Transition (same op over [M, D] rows): LN kernel + two MFMA GEMMs.
 * Replaces Transition.forward (transition.py:52-91) for the single
 * representation s and any width / hidden / output width the fused row kernel
 * does not take, including out_dim != D (the denoiser's token/atom mixers,
 * Transition(dim=a_s+atom_s, out_dim=atom_s or a_s, use_norm=False),
 * diffusion.py:623-634).  D a multiple of 16; hidden and out_dim multiples of
 * 32.  x: [M, D]; fc1_w, fc2_w: [hidden, D]; fc3_w: [out_dim, hidden];
 * out: [M, out_dim].  residual=1 needs out_dim == D.
 * res_tail: NULL or the [M, D] int8 tail of the residual stream (residual=1).
 */
size_t bioemu_transition_token_workspace_bytes(int64_t M, int64_t D, int64_t hidden);
int bioemu_transition_token_fwd(const void* x, const float* norm_w, const float* norm_b,
                                const void* fc1_w, const void* fc2_w, const void* fc3_w, void* out,
                                int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t M, int64_t D,
                                int64_t hidden, int64_t out_dim, int use_norm, int residual, hipStream_t stream);

/*
 * Pair-weighted averaging (MSA module), fused: LN_m -> v = Wm m', g = sigmoid(Wg m');
 * w = softmax_j(LN_z(z) Wz^T, keys with mask 0 replaced by -1e6);
 * o[s,i,h] = sum_j w[h,i,j] v[s,j,h];  out = (g * o) Wo^T (+ m when residual).
 * Replaces PairWeightedAveraging.forward
 * (src/bioemu2/biomoa/ops/pair_weighted_averaging.py:59-154; both of its
 * chunk_heads paths compute these values).  m, out: [B, S, N, c_m] bf16 (out
 * may equal m when residual != 0); z: [B, N, N, c_z] bf16; mask: [B, N, N]
 * uint8.  norm_z_b may be null (use_bias_in_layer_norm=False).  Supported:
 * c_m = 64, c_z = 128, c_h = 32, H = 8, N <= 4096.
 * res_tail: NULL or the [B, S, N, c_m] int8 tail of the residual stream m (residual=1).
 */
size_t bioemu_pwa_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_m, int64_t c_h, int64_t H);
int bioemu_pwa_fwd(const void* m, const void* z, const uint8_t* mask, const float* norm_m_w, const float* norm_m_b,
                   const void* w_m, const void* w_g, const float* norm_z_w, const float* norm_z_b, const void* w_z,
                   const void* w_o, void* out, int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t B, int64_t S,
                   int64_t N, int64_t c_m, int64_t c_z, int64_t c_h, int64_t H, int residual, hipStream_t stream);

/*
 * Attention with pair bias over the single representation.
 * Replaces AttentionPairBias.forward (src/bioemu2/biomoa/ops/attention_pair_bias.py:128-225)
 * with the non-fused bias branch (_proj_z_fused, :114-117):
 *   s' = LN_s(s) (norm_s_w/b null: initial_norm=False);  q,k,v = chunk(s' Wqkv^T); q += q_bias
 *   g = sigmoid(s' Wg^T);  bias = LN_z(z) Wz^T  (norm_z_b may be null)
 *   o = softmax(q k^T / sqrt(d) + bias; keys with mask 0 replaced by -1e6) v
 *   out = (g * o) Wo^T   (+ s when residual != 0)
 * s, out: [B*mult, N, c_s] bf16; z: [B, N, N, c_z] bf16; mask [B, N] uint8.
 * The bias is shared by the `mult` copies of each batch element (multiplicity).
 * Supported: c_z = 128, head dim 24 (c_s = 24*H, c_s in {128, 384}).
 * res_tail: NULL or the [B*mult, N, c_s] int8 tail of the residual stream s (residual=1).
 */
size_t bioemu_apb_workspace_bytes(int64_t B, int64_t mult, int64_t N, int64_t c_s, int64_t H);
int bioemu_apb_fwd(const void* s, const void* z, const uint8_t* mask, const float* norm_s_w,
                   const float* norm_s_b, const void* w_qkv, const float* q_bias, const void* w_g,
                   const float* norm_z_w, const float* norm_z_b, const void* w_z, const void* w_o,
                   void* out, int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t B, int64_t mult,
                   int64_t N, int64_t c_s, int64_t c_z, int64_t H, int residual, hipStream_t stream);

/*
 * Sliding-window attention with pair bias (the denoiser's atom transformer).
 * Replaces AttentionPairBiasSlidingWindow.forward
 * (src/bioemu2/biomoa/ops/attention_pair_bias.py:277-340): the projections of
 * bioemu_apb_fwd per atom; window w of W queries attends to the H keys at atom
 * positions [w*W - (H-W)/2, w*W - (H-W)/2 + H) of the same copy (zero k / v,
 * mask 0 outside [0, NW*W)); bias = LN_z(z) Wz^T per (batch, window), shared
 * by the `mult` copies; masked keys replaced by -1e6.
 * s, out: [B*mult*NW, W, c_s] bf16 (rows ordered batch, copy, window; out may
 * equal s when residual != 0); z: [B, NW, W, H, c_z] bf16; mask: [B*NW, W]
 * uint8.  norm_s_w/b null: initial_norm=False; norm_z_b may be null.
 * Supported: W = 32, H a multiple of 32 with H - W a multiple of 32, head dim
 * 32 (c_s = 32*heads, c_s in {64, 128, 384}), c_z in {16, 32}.
 */
size_t bioemu_swa_workspace_bytes(int64_t B, int64_t mult, int64_t NW, int64_t W, int64_t H, int64_t c_s,
                                  int64_t heads);
int bioemu_swa_fwd(const void* s, const void* z, const uint8_t* mask, const float* norm_s_w,
                   const float* norm_s_b, const void* w_qkv, const float* q_bias, const void* w_g,
                   const float* norm_z_w, const float* norm_z_b, const void* w_z, const void* w_o,
                   void* out, void* workspace, size_t workspace_bytes, int64_t B, int64_t mult,
                   int64_t NW, int64_t W, int64_t H, int64_t c_s, int64_t c_z, int64_t heads, int residual,
                   hipStream_t stream);

/*
 * Distogram head: out[b,i,j,:] = (z[b,i,j] + z[b,j,i]) w^T + b.
 * Replaces DistogramModule.forward (src/bioemu2/biomoa/modules/embedders.py:191-206).
 * z: [B, N, N, c_z] bf16; w: [num_bins, c_z] bf16; b: [num_bins] fp32;
 * out: [B, N, N, num_bins], bf16 (out_f32 = 0) or fp32 (out_f32 = 1: the fp32
 * accumulator plus the bias, unrounded), exactly symmetric in i, j.
 * Supported: c_z = 128, 1 <= num_bins <= 128.
 */
int bioemu_distogram_fwd(const void* z, const void* w, const float* b, void* out, int64_t B, int64_t N,
                         int64_t c_z, int64_t num_bins, int out_f32, hipStream_t stream);

/*
 * PairwiseConditioning input projection: out = LN([z_trunk, rel]) w^T (LayerNorm
 * over the token_z + c_rel concatenated channels, eps 1e-5, no Linear bias).
 * Replaces the dim_pairwise_init_proj step of PairwiseConditioning.forward
 * (src/bioemu2/biomoa/modules/diffusion.py:509-525); its transitions run
 * bioemu_transition_pair_fwd (hidden = 2*a_z) with residual=1.
 * z_trunk, rel: [P, 128] bf16 rows; ln_w, ln_b: [256] fp32; w: [a_z, 256] bf16;
 * out: [P, a_z] bf16; with out_tail (int8 [P, a_z], optional) out is written as
 * a residual stream (bf16 value + int8 tail, the form the transitions' res_tail
 * updates in place).  The workspace holds w with the LayerNorm folded in.
 * Supported: token_z = c_rel = a_z = 128.
 */
size_t bioemu_pair_cond_workspace_bytes(int64_t token_z, int64_t c_rel, int64_t a_z);
int bioemu_pair_cond_proj_fwd(const void* z_trunk, const void* rel, const float* ln_w, const float* ln_b,
                              const void* w, void* out, int8_t* out_tail, void* workspace, size_t workspace_bytes,
                              int64_t P, int64_t token_z, int64_t c_rel, int64_t a_z, hipStream_t stream);

/*
 * Fused OuterProductMean.
 * Replaces OuterProductMeanVanilla.forward / OuterProductMeanTritonMemorySaving.forward
 * (src/bioemu2/biomoa/ops/outer_product_mean.py:45-75, :129-152):
 *   p = proj_ab(LN(m)); p[mask == 0] = 0; a, b = chunk(p, 2)
 *   o[b,i,j,c*C_H+d] = sum_s a[b,s,i,c] b[b,s,j,d] / num_valid[b]   (fp32, mean before the bf16 cast)
 *   out = o Wo^T + b_o   (+ z_res when z_res != NULL; out may equal z_res)
 * m: [B,S,N,c_in] bf16; mask: [B,S,N] uint8.  mean_rows=1 divides by
 * num_valid = max(1, #rows with any valid entry) (a [B,S,N] reference mask);
 * mean_rows=0 divides by 1 (a [B,N] reference mask, expanded over S by the caller).
 * w_ab: [2*C_H, c_in]; w_o: [c_out, C_H*C_H]; b_o: [c_out] fp32; out: [B,N,N,c_out] bf16.
 * Supported: c_in = 64, C_H = 32, c_out = 128.
 * res_tail: NULL or the [B,N,N,c_out] int8 tail of the residual stream z_res (needs z_res).
 */
size_t bioemu_opm_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_in, int64_t c_hidden);
int bioemu_opm_fwd(const void* m, const uint8_t* mask, int mean_rows, const float* norm_w,
                   const float* norm_b, const void* w_ab, const void* w_o, const float* b_o,
                   const void* z_res, void* out, int8_t* res_tail, void* workspace, size_t workspace_bytes, int64_t B,
                   int64_t S, int64_t N, int64_t c_in, int64_t c_hidden, int64_t c_out,
                   hipStream_t stream);

/*
 * Residual-stream conversion (no counterpart in the reference, whose bf16
 * trunk stores z and s as plain bf16; see "Residual tails" above).
 * split: x (n fp32) -> hi (n bf16, round to nearest) + tail (n int8).
 * join:  hi + tail -> out (n fp32).  n a multiple of 16; 16-byte aligned buffers.
 */
int bioemu_stream_split(const float* x, void* hi, int8_t* tail, int64_t n, hipStream_t stream);
int bioemu_stream_join(const void* hi, const int8_t* tail, float* out, int64_t n, hipStream_t stream);

/*
 * Trunk recycling update, pair form: out = base + W LN(x) over P rows of 128
 * channels.  Replaces `z = z_init + self.z_recycle(self.z_norm(z))`
 * (src/bioemu2/biomoa/modules/pairmixer.py:282-283; LayerNorm(token_z) and
 * Linear(token_z, token_z, bias=False) at :186-191).  x, base, out bf16
 * [P][128]; norm_w/norm_b fp32 [128]; W bf16 [128][128].  base_tail / out_tail
 * (int8, optional, independently) carry base and out as residual streams.
 * out may alias x or base.  workspace: bioemu_pair_ln_linear_workspace_bytes.
 */
size_t bioemu_pair_ln_linear_workspace_bytes(int64_t Dc);
int bioemu_pair_ln_linear_fwd(const void* x, const float* norm_w, const float* norm_b, const void* w,
                              const void* base, const int8_t* base_tail, void* out, int8_t* out_tail,
                              void* workspace, size_t workspace_bytes, int64_t P, int64_t Dc, hipStream_t stream);

/*
 * Trunk recycling update, token form: out = base + W LN(x) over M rows of Dc
 * channels (Dc a multiple of 32).  Replaces `s = s_init + self.s_recycle(
 * self.s_norm(s))` (pairmixer.py:281; LayerNorm(token_s), Linear(token_s,
 * token_s, bias=False) at :186-190).  base_tail and out_tail (int8) are both
 * given or both NULL; out may alias x.  workspace: *_workspace_bytes(M, Dc).
 */
size_t bioemu_token_ln_linear_workspace_bytes(int64_t M, int64_t Dc);
int bioemu_token_ln_linear_fwd(const void* x, const float* norm_w, const float* norm_b, const void* w,
                               const void* base, const int8_t* base_tail, void* out, int8_t* out_tail,
                               void* workspace, size_t workspace_bytes, int64_t M, int64_t Dc, hipStream_t stream);

/*
 * Trunk unconditional branch (classifier-free guidance): out = z_init +
 * uncond_transition(z_norm(z_init)).  Replaces `z = z_init + self.uncond_
 * transition(self.z_norm(z_init))` (PairMixerSequenceEmbedder.forward,
 * src/bioemu2/biomoa/modules/pairmixer.py:266-273; z_norm = LayerNorm(token_z)
 * at :190, uncond_transition = Transition(token_z, 4 token_z) at :194-200,
 * transition.py:52-91).  z_init, out bf16 [P][128]; z_norm_w/b and the
 * transition's norm.weight/bias t_norm_w/b fp32 [128]; fc1_w, fc2_w bf16
 * [hidden][128]; fc3_w bf16 [128][hidden]; hidden = 512 or 256.  z_init_tail /
 * out_tail (int8 [P][128]) carry z_init and out as residual streams, both given
 * or both NULL; the LayerNorm reads z_init's bf16 part.  out may alias z_init
 * (then out_tail must be z_init_tail).  workspace: *_workspace_bytes(P, 128, hidden).
 */
size_t bioemu_trunk_uncond_workspace_bytes(int64_t P, int64_t Dc, int64_t hidden);
int bioemu_trunk_uncond_fwd(const void* z_init, const int8_t* z_init_tail, const float* z_norm_w,
                            const float* z_norm_b, const float* t_norm_w, const float* t_norm_b, const void* fc1_w,
                            const void* fc2_w, const void* fc3_w, void* out, int8_t* out_tail, void* workspace,
                            size_t workspace_bytes, int64_t P, int64_t Dc, int64_t hidden, hipStream_t stream);

/*
 * MSA input embedding.  Replaces PairMixerMSAModule.forward's
 *   m = msa_proj(cat(msa, has_deletion, deletion_value[, msa_paired])) + s_proj(emb)[:, None]
 * (pairmixer.py:591-599; bias-free Linear layers at :527-532).  msa fp32
 * [B][R][T][F0]; has_deletion, deletion_value, msa_paired (optional) fp32
 * [B][R][T]; emb fp32 [B][T][E]; w_msa fp32 [msa_s][F0 + 2 (+1)]; w_s fp32
 * [msa_s][E]; msa_s = 64, F0 + 3 <= 64.  m is written as the MSA residual
 * stream: bf16 [B][R][T][64] plus its int8 tail.  Computed in fp32.
 * workspace: bioemu_msa_embed_workspace_bytes(B, T).
 */
size_t bioemu_msa_embed_workspace_bytes(int64_t B, int64_t T);
int bioemu_msa_embed_fwd(const float* msa, const float* has_deletion, const float* deletion_value,
                         const float* msa_paired, const float* emb, const float* w_msa, const float* w_s, void* m,
                         int8_t* m_tail, void* workspace, size_t workspace_bytes, int64_t B, int64_t R, int64_t T,
                         int64_t F0, int64_t E, int64_t msa_s, hipStream_t stream);

/*
 * fp32 arithmetic (fp32 operands, fp32 MFMA accumulation, fp32 softmax) for the
 * ops the reference's denoiser runs with autocast off (src/bioemu2/biomoa/
 * models/score_model.py:355, model.py:387).  Same arguments and semantics as the
 * bf16 entry points above, with every activation, weight and output fp32:
 *   bioemu_apb_fwd_f32       AttentionPairBias.forward (attention_pair_bias.py:128-225);
 *                            head dim 24 or 32, c_s a multiple of 32, c_z in {16, 32, 128}.
 *   bioemu_swa_fwd_f32       AttentionPairBiasSlidingWindow.forward (:277-340); W = 32,
 *                            H a multiple of 32, head dim 32.
 *   bioemu_transition_fwd_f32  Transition.forward (transition.py:52-91) on M rows:
 *                            dim a multiple of 8, hidden and out_dim multiples of 32.
 *   bioemu_pair_cond_proj_fwd_f32  the LayerNorm + LinearNoBias of PairwiseConditioning
 *                            (biomoa/modules/diffusion.py:521-524) over P pair rows: the
 *                            concatenation [z_trunk row | rel row] is read in place;
 *                            token_z + c_rel a multiple of 8, a_z of 32.  Its transitions
 *                            (:526-527) are bioemu_transition_fwd_f32 with residual=1.
 *   bioemu_trimul_fwd_f32    the triangle multiplicative update in IEEE fp32, for a trunk run
 *                            with autocast off (TriangleMultiplicationFull.forward,
 *                            triangle_multiplication.py:89-99; TriangleMultiplicationCueq with
 *                            its default matmul_precision="ieee", :104-125): the arguments of
 *                            bioemu_trimul_fwd without res_tail; dim a multiple of 32,
 *                            B * dim <= 65535.
 *   bioemu_opm_fwd_f32       OuterProductMeanVanilla.forward (outer_product_mean.py:45-75) in
 *                            IEEE fp32 for a trunk run with autocast off: the arguments of
 *                            bioemu_opm_fwd as fp32 without res_tail (out = OPM(m) + z_res when
 *                            z_res is given); c_hidden = 32, c_in a multiple of 8, c_out of 32.
 *                            Its workspace holds the [B, N, N, 32 * 32] outer-product means.
 *   bioemu_pwa_fwd_f32       PairWeightedAveraging.forward (pair_weighted_averaging.py:59-154)
 *                            in IEEE fp32: the arguments of bioemu_pwa_fwd as fp32 without
 *                            res_tail, plus the masking constant inf (the module's inf; masked
 *                            logits become -inf); c_h = 32, c_m a multiple of 32, c_z 16, 32 or
 *                            128, B * H <= 65535.
 *   bioemu_msa_embed_fwd_f32 bioemu_msa_embed_fwd writing m as fp32 (no tail).
 *   bioemu_ln_linear_fwd_f32 out = (base +) LN(x) W^T over M rows (x [M][K], w [N][K]; base
 *                            may be null): the recycling updates of the trunk
 *                            (pairmixer.py:276-283), replacing bioemu_pair_ln_linear_fwd and
 *                            bioemu_token_ln_linear_fwd; K a multiple of 8, N of 32.
 *   bioemu_trunk_uncond_fwd_f32  bioemu_trunk_uncond_fwd in fp32 (z_init + uncond_transition(
 *                            z_norm(z_init)), :266-273); dim and hidden multiples of 32.
 *   bioemu_distogram_fwd_f32 DistogramModule.forward (embedders.py:191-206) on fp32 z:
 *                            (z + z^T) W^T + b; c_z a multiple of 8, num_bins of 32.
 *   bioemu_triatt_fwd_f32    triangle attention (no counterpart in the reference, as
 *                            bioemu_triatt_fwd) in fp32: the arguments of bioemu_triatt_fwd
 *                            as fp32 without res_tail; D = 32 or 128 with heads of 32
 *                            channels, B * N <= 65535.
 * Residual tails do not apply (the stream is fp32).
 */
size_t bioemu_apb_f32_workspace_bytes(int64_t B, int64_t mult, int64_t N, int64_t c_s, int64_t H);
int bioemu_apb_fwd_f32(const float* s, const float* z, const uint8_t* mask, const float* norm_s_w,
                       const float* norm_s_b, const float* w_qkv, const float* q_bias, const float* w_g,
                       const float* norm_z_w, const float* norm_z_b, const float* w_z, const float* w_o, float* out,
                       void* workspace, size_t workspace_bytes, int64_t B, int64_t mult, int64_t N, int64_t c_s,
                       int64_t c_z, int64_t H, int residual, hipStream_t stream);
size_t bioemu_swa_f32_workspace_bytes(int64_t B, int64_t mult, int64_t NW, int64_t W, int64_t H, int64_t c_s,
                                      int64_t heads);
int bioemu_swa_fwd_f32(const float* s, const float* z, const uint8_t* mask, const float* norm_s_w,
                       const float* norm_s_b, const float* w_qkv, const float* q_bias, const float* w_g,
                       const float* norm_z_w, const float* norm_z_b, const float* w_z, const float* w_o, float* out,
                       void* workspace, size_t workspace_bytes, int64_t B, int64_t mult, int64_t NW, int64_t W,
                       int64_t H, int64_t c_s, int64_t c_z, int64_t heads, int residual, hipStream_t stream);
size_t bioemu_transition_f32_workspace_bytes(int64_t M, int64_t Dc, int64_t hidden);
int bioemu_transition_fwd_f32(const float* x, const float* norm_w, const float* norm_b, const float* fc1_w,
                              const float* fc2_w, const float* fc3_w, float* out, void* workspace,
                              size_t workspace_bytes, int64_t M, int64_t Dc, int64_t hidden, int64_t out_dim,
                              int use_norm, int residual, hipStream_t stream);
size_t bioemu_pair_cond_f32_workspace_bytes(int64_t P, int64_t token_z, int64_t c_rel);
int bioemu_pair_cond_proj_fwd_f32(const float* z_trunk, const float* rel, const float* ln_w, const float* ln_b,
                                  const float* w, float* out, void* workspace, size_t workspace_bytes, int64_t P,
                                  int64_t token_z, int64_t c_rel, int64_t a_z, hipStream_t stream);
size_t bioemu_trimul_f32_workspace_bytes(int64_t B, int64_t N, int64_t Dc);
int bioemu_trimul_fwd_f32(const float* x, const uint8_t* mask, const float* norm_in_w, const float* norm_in_b,
                          const float* p_in_w, const float* g_in_w, const float* norm_out_w, const float* norm_out_b,
                          const float* p_out_w, const float* g_out_w, float* out, void* workspace,
                          size_t workspace_bytes, int64_t B, int64_t N, int64_t Dc, int outgoing, int residual,
                          hipStream_t stream);
size_t bioemu_opm_f32_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_in, int64_t c_hidden);
int bioemu_opm_fwd_f32(const float* m, const uint8_t* mask, int mean_rows, const float* norm_w, const float* norm_b,
                       const float* w_ab, const float* w_o, const float* b_o, const float* z_res, float* out,
                       void* workspace, size_t workspace_bytes, int64_t B, int64_t S, int64_t N, int64_t c_in,
                       int64_t c_hidden, int64_t c_out, hipStream_t stream);
size_t bioemu_pwa_f32_workspace_bytes(int64_t B, int64_t S, int64_t N, int64_t c_m, int64_t c_h, int64_t H);
int bioemu_pwa_fwd_f32(const float* m, const float* z, const uint8_t* mask, const float* norm_m_w,
                       const float* norm_m_b, const float* norm_z_w, const float* norm_z_b, const float* w_m,
                       const float* w_g, const float* w_z, const float* w_o, float* out, void* workspace,
                       size_t workspace_bytes, int64_t B, int64_t S, int64_t N, int64_t c_m, int64_t c_z,
                       int64_t c_h, int64_t H, float inf, int residual, hipStream_t stream);
int bioemu_msa_embed_fwd_f32(const float* msa, const float* has_deletion, const float* deletion_value,
                             const float* msa_paired, const float* emb, const float* w_msa, const float* w_s,
                             float* m, void* workspace, size_t workspace_bytes, int64_t B, int64_t R, int64_t T,
                             int64_t F0, int64_t E, int64_t msa_s, hipStream_t stream);
size_t bioemu_ln_linear_f32_workspace_bytes(int64_t M, int64_t K);
int bioemu_ln_linear_fwd_f32(const float* x, const float* norm_w, const float* norm_b, const float* w,
                             const float* base, float* out, void* workspace, size_t workspace_bytes, int64_t M,
                             int64_t K, int64_t N, hipStream_t stream);
size_t bioemu_trunk_uncond_f32_workspace_bytes(int64_t P, int64_t Dc, int64_t hidden);
int bioemu_trunk_uncond_fwd_f32(const float* z_init, const float* z_norm_w, const float* z_norm_b,
                                const float* t_norm_w, const float* t_norm_b, const float* fc1_w, const float* fc2_w,
                                const float* fc3_w, float* out, void* workspace, size_t workspace_bytes, int64_t P,
                                int64_t Dc, int64_t hidden, hipStream_t stream);
size_t bioemu_distogram_f32_workspace_bytes(int64_t B, int64_t N, int64_t c_z);
int bioemu_distogram_fwd_f32(const float* z, const float* w, const float* b, float* out, void* workspace,
                             size_t workspace_bytes, int64_t B, int64_t N, int64_t c_z, int64_t num_bins,
                             hipStream_t stream);
size_t bioemu_triatt_f32_workspace_bytes(int64_t B, int64_t N, int64_t D, int64_t H);
int bioemu_triatt_fwd_f32(const float* z, const uint8_t* mask, const float* norm_w, const float* norm_b,
                          const float* w_proj, const float* w_o, float* out, void* workspace, size_t workspace_bytes,
                          int64_t B, int64_t N, int64_t D, int64_t H, int starting, int residual, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BIOEMU2_MI355X_H */
