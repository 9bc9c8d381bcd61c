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
//   triatt_proj  : LN + all five projections (q, k, v, g, bias) on MFMA with
//                  weights staged once per workgroup in LDS; writes the frame-
//                  ordered operands of the attention and a frame-ordered mask.
//   triatt_flash : per (b, row i, 32 queries) online-softmax attention over
//                  all keys, 4 heads, with the gate and the output projection
//                  fused in the epilogue and the residual added in place.
// H = 4 heads of d = 32 over c = 128 channels.
#include <algorithm>

#include "common.h"
#include "internal.h"
#include "pairtile.h"

namespace bioemu {
namespace {

constexpr int C = 128;
constexpr int H = 4;
constexpr int DH = 32;
constexpr int kProjRows = 4 * C + H;       // q, k, v, g, bias rows of the packed weight
constexpr int kProjRowsPad = 4 * C + 32;   // bias block padded to one 32-row MFMA block
constexpr int kProjThreads = 512;
constexpr int kProjSmem = kProjRowsPad * kLdw * 2;
constexpr int kFlashThreads = 256;         // 4 waves x 32 queries = 128 queries per workgroup

struct TriAttBuffers {
  bf16* q;       // [B][Np][Np][C]  frame-ordered, pair-major
  bf16* k;       // [B][Np][Np][C]
  bf16* g;       // [B][Np][Np][C]  sigmoid already applied
  bf16* vt;      // [B][Np][C][Np]  channel-major per frame row
  bf16* bias;    // [B][H][Np][Np]
  uint8_t* mask; // [B][Np][Np]     frame-ordered 0/1 (0 outside [0, N))
};

// ---------------------------------------------------------------------------
// Projection kernel.  Tile = (b, frame row i, 32 frame columns).
// ---------------------------------------------------------------------------
template <bool kStarting>
__global__ __launch_bounds__(kProjThreads) void triatt_proj_kernel(
    const bf16* __restrict__ z, const uint8_t* __restrict__ mask, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ w, TriAttBuffers buf, int B, int N,
    int Np) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* wl = reinterpret_cast<bf16*>(smem);
  stage_weights(wl, w, kProjRows, kProjRowsPad);
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rho = lane & 31, h = lane >> 5;
  const int waves = blockDim.x >> 6;
  const int tiles_per_row = Np / 32;
  const long long ntiles = (long long)B * Np * tiles_per_row;
  const size_t plane = (size_t)Np * Np;

  for (long long t = (long long)blockIdx.x * waves + wave; t < ntiles; t += (long long)gridDim.x * waves) {
    const int kt = (int)(t % tiles_per_row);
    const int i = (int)((t / tiles_per_row) % Np);
    const int b = (int)(t / ((long long)tiles_per_row * Np));
    const int k0 = kt * 32;

    // This lane's pair slot: frame (i, k0 + perm32(rho)).
    const int kk = k0 + perm32(rho);
    const bool valid = i < N && kk < N;
    const size_t zpair = kStarting ? ((size_t)b * N + i) * N + kk : ((size_t)b * N + kk) * N + i;
    bf16x8 raw[8], x[8];
    load_half_row(z + zpair * C, h, valid, raw);
    layernorm_half_row(raw, ln_w, ln_b, h, 1e-5f, x);

    const size_t frow = ((size_t)b * Np + i) * Np;  // frame row base (pairs)
    // q, k, g: pair-major.  Lane (n, h) holds pair slot perm32(rho), channels cb*32+16h..+15.
    const size_t pm_off = (frow + kk) * C;
#pragma unroll 1
    for (int cb = 0; cb < 4; ++cb) {
      f32x16 aq = proj_block_pm(x, wl, 0 * C + cb * 32, rho, h);
      float vq[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) vq[u] = aq[u];
      store16(buf.q + pm_off + cb * 32 + 16 * h, vq);
      f32x16 ak = proj_block_pm(x, wl, 1 * C + cb * 32, rho, h);
#pragma unroll
      for (int u = 0; u < 16; ++u) vq[u] = ak[u];
      store16(buf.k + pm_off + cb * 32 + 16 * h, vq);
      f32x16 ag = proj_block_pm(x, wl, 3 * C + cb * 32, rho, h);
#pragma unroll
      for (int u = 0; u < 16; ++u) vq[u] = sigmoidf_fast(ag[u]);
      store16(buf.g + pm_off + cb * 32 + 16 * h, vq);
    }
    // v^T: channel-major.  Lane (n, h) holds channel cb*32+n, pairs k0+16h..+15.
#pragma unroll 1
    for (int cb = 0; cb < 4; ++cb) {
      f32x16 av = proj_block_cm(x, wl, 2 * C + cb * 32, rho, h);
      float vv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) vv[u] = av[u];
      store16(buf.vt + (((size_t)b * Np + i) * C + cb * 32 + rho) * Np + k0 + 16 * h, vv);
    }
    {
      f32x16 ab = proj_block_cm(x, wl, 4 * C, rho, h);
      if (rho < H) {
        float vb[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) vb[u] = ab[u];
        store16(buf.bias + ((size_t)b * H + rho) * plane + (size_t)i * Np + k0 + 16 * h, vb);
      }
    }
    if (h == 0) {
      const int kc = k0 + rho;
      uint8_t mv = 0;
      if (i < N && kc < N) {
        const size_t mp = kStarting ? ((size_t)b * N + i) * N + kc : ((size_t)b * N + kc) * N + i;
        mv = mask[mp] != 0;
      }
      buf.mask[frow + kc] = mv;
    }
  }
}

// ---------------------------------------------------------------------------
// Flash attention kernel.  Workgroup = (b, frame row i, 128 queries);
// wave w owns queries q0 = 128*blockIdx.x + 32w, all 4 heads.
//
// S^T = K Q^T per head: A = K (pair slot rho <-> key k0 + perm32(rho)),
// B = Q^T (lane n <-> query q0 + n).  D lane (n, hh) register u <-> key
// k0 + 16hh + u, so a lane holds 16 consecutive keys of one query; the row
// max / sum need one cross-half shuffle.  O^T = V^T P^T: A = V^T (slot rho <->
// d = perm32(rho)), B = P^T straight from the softmax registers (k-step s,
// half hh, t <-> key k0 + 16hh + 8s + t).  D lane (n, hh) register u <->
// d = 16hh + u.  The epilogue feeds g*o back as the B operand of
// update^T = Wo (g*o)^T, again without leaving registers.
// ---------------------------------------------------------------------------
template <bool kStarting>
__global__ __launch_bounds__(kFlashThreads) void triatt_flash_kernel(
    TriAttBuffers buf, const bf16* __restrict__ wo, const bf16* zres, bf16* out, int N, int Np,
    int residual) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int b = blockIdx.z, i = blockIdx.y;
  const int q0 = blockIdx.x * 128 + wave * 32;
  if (q0 >= Np) return;  // no barriers in this kernel

  const size_t frow = ((size_t)b * Np + i) * Np;
  const size_t plane = (size_t)Np * Np;
  const float qk_scale = 0.17677669529663687f * kLog2e;  // log2(e) / sqrt(32)
  const float masked_logit = -1e6f * kLog2e;

  // Q^T fragments (B operand): lane (n, hh), step s: d = 16s + 8hh + t.
  bf16x8 qf[H][2];
  {
    const bf16* qrow = buf.q + (frow + q0 + n) * C;
#pragma unroll
    for (int hd = 0; hd < H; ++hd)
#pragma unroll
      for (int s = 0; s < 2; ++s) qf[hd][s] = load8(qrow + hd * DH + 16 * s + 8 * hh);
  }

  f32x16 o[H];
  float m[H], l[H];
#pragma unroll
  for (int hd = 0; hd < H; ++hd) {
    o[hd] = zero16();
    m[hd] = -INFINITY;
    l[hd] = 0.f;
  }

  const bf16* krow = buf.k + frow * C;
  const bf16* vrow = buf.vt + ((size_t)b * Np + i) * C * Np;
  const uint8_t* mrow = buf.mask + frow;

  for (int k0 = 0; k0 < Np; k0 += 32) {
    // Key mask of this lane's 16 keys k0 + 16hh + u.
    const uint4 mk = *reinterpret_cast<const uint4*>(mrow + k0 + 16 * hh);
    const uint32_t mw[4] = {mk.x, mk.y, mk.z, mk.w};
    const int kslot = k0 + perm32(n);  // key row of this lane as an A operand
#pragma unroll
    for (int hd = 0; hd < H; ++hd) {
      const bf16* kp = krow + (size_t)kslot * C + hd * DH + 8 * hh;
      f32x16 s = zero16();
      s = mfma32(load8(kp), qf[hd][0], s);
      s = mfma32(load8(kp + 16), qf[hd][1], s);

      const bf16* bp = buf.bias + ((size_t)b * H + hd) * plane + (size_t)(q0 + n) * Np + k0 + 16 * hh;
      const bf16x8 b0 = load8(bp), b1 = load8(bp + 8);
      float t[16];
      float bmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float bv = bf2f(u < 8 ? b0[u] : b1[u - 8]);
        float x = s[u] * qk_scale + bv * kLog2e;
        const bool valid_key = ((mw[u >> 2] >> (8 * (u & 3))) & 0xff) != 0;
        if (!valid_key) x = masked_logit;
        if (k0 + 16 * hh + u >= N) x = -INFINITY;
        t[u] = x;
        bmax = fmaxf(bmax, x);
      }
      bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
      const float m_new = fmaxf(m[hd], bmax);
      const float alpha = fast_exp2(m[hd] - m_new);
      m[hd] = m_new;
      float psum = 0.f;
      bf16x8 pb[2];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float p = fast_exp2(t[u] - m_new);
        psum += p;
        pb[u >> 3][u & 7] = f2bf(p);
      }
      l[hd] = l[hd] * alpha + psum;
#pragma unroll
      for (int u = 0; u < 16; ++u) o[hd][u] *= alpha;

      const bf16* vp = vrow + (size_t)(hd * DH + perm32(n)) * Np + k0 + 16 * hh;
      o[hd] = mfma32(load8(vp), pb[0], o[hd]);
      o[hd] = mfma32(load8(vp + 8), pb[1], o[hd]);
    }
  }

  // Epilogue: normalise, gate, output projection, residual.
  bf16x8 gob[8];
  {
    const bf16* grow = buf.g + (frow + q0 + n) * C;
#pragma unroll
    for (int hd = 0; hd < H; ++hd) {
      const float lt = l[hd] + __shfl_xor(l[hd], 32);
      const float inv = 1.0f / lt;
      const bf16x8 g0 = load8(grow + hd * DH + 16 * hh);
      const bf16x8 g1 = load8(grow + hd * DH + 16 * hh + 8);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        gob[2 * hd][u] = f2bf(bf2f(g0[u]) * (o[hd][u] * inv));
        gob[2 * hd + 1][u] = f2bf(bf2f(g1[u]) * (o[hd][8 + u] * inv));
      }
    }
  }
  const int q = q0 + n;
  const bool store = q < N;
  const size_t zpair = kStarting ? ((size_t)b * N + i) * N + q : ((size_t)b * N + q) * N + i;
#pragma unroll 1
  for (int cb = 0; cb < 4; ++cb) {
    f32x16 acc = zero16();
    const bf16* wrow = wo + (size_t)(cb * 32 + perm32(n)) * C + 16 * hh;
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = mfma32(load8(wrow + 32 * (s >> 1) + 8 * (s & 1)), gob[s], acc);
    if (store) {
      const size_t off = zpair * C + cb * 32 + 16 * hh;
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = acc[u];
      if (residual) {
        const bf16x8 r0 = load8(zres + off), r1 = load8(zres + off + 8);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          v[u] += bf2f(r0[u]);
          v[8 + u] += bf2f(r1[u]);
        }
      }
      store16(out + off, v);
    }
  }
}

}  // namespace
}  // namespace bioemu

using namespace bioemu;

static size_t triatt_np(int64_t N) { return (size_t)round_up(N, 32); }

extern "C" size_t bioemu_triatt_workspace_bytes(int64_t B, int64_t N, int64_t Dc, int64_t Hc) {
  if (B <= 0 || N <= 0 || Dc != C || Hc != H) return 0;
  const size_t Np = triatt_np(N);
  const size_t pairs = (size_t)B * Np * Np;
  // q, k, g, v^T (bf16 x C each) + bias (bf16 x H) + mask (u8), each 256-byte aligned
  return round_up(pairs * C * 2, 256) * 4 + round_up(pairs * H * 2, 256) + round_up(pairs, 256);
}

extern "C" int bioemu_triatt_fwd(const void* z, const uint8_t* mask, const float* norm_w,
                                 const float* norm_b, const void* w_proj, const void* w_o, void* out,
                                 void* workspace, size_t workspace_bytes, int64_t B, int64_t N,
                                 int64_t Dc, int64_t Hc, int starting, int residual,
                                 hipStream_t stream) {
  if (Dc != C || Hc != H)
    return set_error(BIOEMU_ERR_UNSUPPORTED, "triatt: only c=128 with 4 heads of 32 is supported (got c=%lld H=%lld)",
                     (long long)Dc, (long long)Hc);
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
  buf.q = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * C * 2, 256);
  buf.k = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * C * 2, 256);
  buf.g = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * C * 2, 256);
  buf.vt = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * C * 2, 256);
  buf.bias = reinterpret_cast<bf16*>(p);
  p += round_up(pairs * H * 2, 256);
  buf.mask = reinterpret_cast<uint8_t*>(p);

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
                         static_cast<const bf16*>(z), mask, norm_w, norm_b, static_cast<const bf16*>(w_proj),
                         buf, (int)B, (int)N, (int)Np);
    else
      hipLaunchKernelGGL(triatt_proj_kernel<false>, dim3(grid1), dim3(kProjThreads), kProjSmem, stream,
                         static_cast<const bf16*>(z), mask, norm_w, norm_b, static_cast<const bf16*>(w_proj),
                         buf, (int)B, (int)N, (int)Np);
  }
  int rc = check_launch("triatt_proj");
  if (rc) return rc;

  dim3 g2((unsigned)((Np + 127) / 128), (unsigned)N, (unsigned)B);
  {
    KernelTimerScope timed("triatt_flash", stream);
    if (starting)
      hipLaunchKernelGGL(triatt_flash_kernel<true>, g2, dim3(kFlashThreads), 0, stream, buf,
                         static_cast<const bf16*>(w_o), static_cast<const bf16*>(z), static_cast<bf16*>(out),
                         (int)N, (int)Np, residual);
    else
      hipLaunchKernelGGL(triatt_flash_kernel<false>, g2, dim3(kFlashThreads), 0, stream, buf,
                         static_cast<const bf16*>(w_o), static_cast<const bf16*>(z), static_cast<bf16*>(out),
                         (int)N, (int)Np, residual);
  }
  return check_launch("triatt_flash");
}
