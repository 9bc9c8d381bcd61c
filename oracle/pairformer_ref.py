"""float32 CPU restatement of the Pairformer hot-path ops (test infrastructure only).

All citations are ``path:line`` inside the reference repository
itsawesomeabhishek/bioemu2 (``src/bioemu2/biomoa/...``).  The arithmetic is
plain float32 PyTorch on the CPU; nothing here runs on, or is shipped to, the
GPU product path.

Parameter dicts use the reference modules' ``state_dict`` keys.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

__all__ = [
    "trimul",
    "triangle_attention",
    "attention_pair_bias",
    "outer_product_mean",
    "pair_weighted_averaging",
    "transition",
    "pairformer_block",
    "pairmixer_layer",
    "pairmixer_msa_layer",
    "pair_mask_from_token_mask",
    "ln_linear",
    "msa_embed",
    "pairmixer_module",
    "pairmixer_msa_module",
    "pairmixer_trunk",
    "pairmixer_uncond",
]


def _f32(t: Tensor) -> Tensor:
    return t.detach().to(device="cpu", dtype=torch.float32)


def _p(params: dict, key: str) -> Tensor:
    return _f32(params[key])


def _ln(x: Tensor, params: dict, prefix: str, eps: float = 1e-5) -> Tensor:
    w = _p(params, prefix + ".weight")
    b = _p(params, prefix + ".bias") if (prefix + ".bias") in params else None
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def pair_mask_from_token_mask(token_mask: Tensor) -> Tensor:
    """``pair_mask = mask_i & mask_j`` (biomoa/modules/pairmixer.py:263-264)."""
    m = token_mask.bool()
    return m.unsqueeze(-1) & m.unsqueeze(-2)


# ----------------------------------------------------------------------------
# Triangle multiplicative update
# ----------------------------------------------------------------------------
def trimul(x: Tensor, mask: Tensor, params: dict, mode: str = "outgoing") -> Tensor:
    """TriangleMultiplicationFull.forward (biomoa/ops/triangle_multiplication.py:89-99).

    Parameters: ``_TriMulBase.__init__`` (triangle_multiplication.py:62-76) —
    norm_in (LN, eps 1e-5), p_in/g_in Linear(D->2D, no bias), norm_out (LN),
    p_out/g_out Linear(D->D, no bias).

    x [B,N,N,D], mask [B,N,N] -> [B,N,N,D] (float32).  The output is not masked.
    """
    if mode not in ("outgoing", "incoming"):
        raise AssertionError(mode)
    x = _f32(x)
    xn = _ln(x, params, "norm_in")  # :90
    proj = (xn @ _p(params, "p_in.weight").T) * torch.sigmoid(
        xn @ _p(params, "g_in.weight").T
    )  # :92
    proj = proj.masked_fill(~mask.bool().unsqueeze(-1), 0.0)  # :93
    a, b = proj.chunk(2, dim=-1)  # :94 (a = channels 0..D-1)
    if mode == "outgoing":
        out = torch.einsum("bikd,bjkd->bijd", a, b)  # :96
    else:
        out = torch.einsum("bkid,bkjd->bijd", a, b)  # :98
    on = _ln(out, params, "norm_out")
    return (on @ _p(params, "p_out.weight").T) * torch.sigmoid(
        xn @ _p(params, "g_out.weight").T
    )  # :99


# ----------------------------------------------------------------------------
# Triangle attention (NOT in the reference: AF3 supplement Alg. 14/15)
# ----------------------------------------------------------------------------
TRIATT_INF = 1e6


def triangle_attention(
    z: Tensor,
    mask: Tensor,
    params: dict,
    num_heads: int = 4,
    starting: bool = True,
    inf: float = TRIATT_INF,
    row_chunk: int | None = None,
) -> Tensor:
    """Triangle attention around the starting (Alg. 14) or ending (Alg. 15) node.

    The reference has no triangle attention (biomoa/modules/pairmixer.py:459-462
    removes it); this restates AlphaFold3 supplement Alg. 14/15 with
    LinearNoBias projections and the reference's masking convention for
    attention: masked keys are *replaced* by ``-inf`` (``masked_fill``), as in
    AttentionPairBias.forward (biomoa/ops/attention_pair_bias.py:184-190).

    Starting node, per batch b, row i, head h:
        zn = LN(z);  q,k,v,g = LinearNoBias(zn) (g through a sigmoid)
        bias[h,j,k] = LinearNoBias(zn)[j,k,h]
        logit[j,k] = q[i,j]·k[i,k]/sqrt(d) + bias[h,j,k];  masked_fill(~mask[i,k], -inf)
        o[i,j] = sum_k softmax_k(logit[j,k]) v[i,k]
        out = LinearNoBias(g ⊙ o)
    Ending node = starting node applied to z^T (mask^T), output transposed back.

    Keys: norm.{weight,bias}, proj_q/k/v/g.weight [H*d, c], proj_b.weight [H, c],
    proj_o.weight [c, H*d].
    """
    z = _f32(z)
    m = mask.bool()
    if not starting:
        z = z.transpose(1, 2)
        m = m.transpose(1, 2)
    B, N, _, _ = z.shape
    H = num_heads
    zn = _ln(z, params, "norm")
    wq, wk, wv = (_p(params, f"proj_{n}.weight") for n in "qkv")
    hd = wq.shape[0]
    d = hd // H
    q = (zn @ wq.T).view(B, N, N, H, d)
    k = (zn @ wk.T).view(B, N, N, H, d)
    v = (zn @ wv.T).view(B, N, N, H, d)
    g = torch.sigmoid(zn @ _p(params, "proj_g.weight").T)
    bias = (zn @ _p(params, "proj_b.weight").T).permute(0, 3, 1, 2)  # [B,H,N(j),N(k)]
    o = torch.empty(B, N, N, H, d)
    chunk = row_chunk or N
    for r0 in range(0, N, chunk):
        r1 = min(N, r0 + chunk)
        # logits [B, rows, H, j, k]
        logit = torch.einsum("brjhd,brkhd->brhjk", q[:, r0:r1], k[:, r0:r1])
        logit = logit / math.sqrt(d) + bias.unsqueeze(1)
        key_mask = m[:, r0:r1][:, :, None, None, :]  # [B, rows, 1, 1, k]
        logit = logit.masked_fill(~key_mask, -inf)
        attn = logit.softmax(dim=-1)
        o[:, r0:r1] = torch.einsum("brhjk,brkhd->brjhd", attn, v[:, r0:r1])
    out = (g * o.reshape(B, N, N, hd)) @ _p(params, "proj_o.weight").T
    if not starting:
        out = out.transpose(1, 2)
    return out.contiguous()


# ----------------------------------------------------------------------------
# Attention with pair bias
# ----------------------------------------------------------------------------
def attention_pair_bias(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    params: dict,
    num_heads: int,
    multiplicity: int = 1,
    initial_norm: bool = True,
    tile_size: int | None = 512,
    inf: float = 1e6,
) -> Tensor:
    """AttentionPairBias.forward (biomoa/ops/attention_pair_bias.py:128-225).

    s [B*M,N,c_s], z [B,N,N,c_z], mask [B,N] bool -> [B*M,N,c_s] (float32).
    Bias = permute(proj_z(norm_z(z))) (``_proj_z_fused`` non-fused branch,
    :114-117); ``norm_z`` has a bias only when its key is present
    (``use_bias_in_layer_norm``, :90).  The core runs query-tiled when
    ``tile_size < N`` (:193-222) exactly as the reference does.
    """
    s = _f32(s)
    z = _f32(z)
    mask = mask.bool().cpu()
    assert s.ndim == 3 and z.ndim == 4 and mask.ndim == 2  # :146
    assert s.shape[0] == z.shape[0] * multiplicity  # :147
    BM, N, c_s = s.shape
    H = num_heads
    d = c_s // H
    if initial_norm:
        s = _ln(s, params, "norm_s")  # :152-153
    qkv = s @ _p(params, "proj_qkv.weight").T  # :156
    q, k, v = qkv.chunk(3, dim=-1)  # :157
    q = (q + _p(params, "proj_q_bias")).view(BM, N, H, d)  # :158
    k = k.view(BM, N, H, d)
    v = v.view(BM, N, H, d)
    g = torch.sigmoid(s @ _p(params, "proj_g.weight").T)  # :161
    zb = _ln(z, params, "norm_z") @ _p(params, "proj_z.weight").T  # :115-116
    z_f = zb.permute(0, 3, 1, 2)  # [B,H,N,N] (:117)
    B_real = z_f.shape[0]
    mask_view = mask.unsqueeze(1).unsqueeze(1)  # [B,1,1,N] (:184)
    chunk = tile_size
    if chunk is None or chunk >= N:
        chunk = N
    o = torch.zeros(BM, N, H, d)
    for qs in range(0, N, chunk):
        qe = min(qs + chunk, N)
        attn = torch.einsum("bchd,bnhd->bhcn", q[:, qs:qe], k)  # :206
        attn = attn / (d**0.5)  # :207
        z_chunk = z_f[..., qs:qe, :]
        attn = (
            attn.view(B_real, multiplicity, *z_chunk.shape[1:]) + z_chunk.unsqueeze(1)
        ).view(attn.shape)  # :209-214
        attn = (
            attn.view(B_real, multiplicity, *attn.shape[1:]).masked_fill(
                ~mask_view.unsqueeze(1), -inf
            )
        ).view(attn.shape)  # :215-220
        attn = attn.softmax(dim=-1)  # :221
        o[:, qs:qe] = torch.einsum("bhcn,bnhd->bchd", attn, v)  # :222
    o = o.reshape(BM, N, c_s)  # :224
    return (g * o) @ _p(params, "proj_o.weight").T  # :225


def sliding_window_keys(num_windows: int, window_queries: int, window_keys: int) -> tuple[Tensor, Tensor]:
    """Absolute key positions of every window and whether they lie in the sequence.

    The key window of size H is centred on the W-query window: it starts
    (H - W) / 2 positions before the window's first query; positions outside
    [0, NW*W) are the reference's zero padding (attention_pair_bias.py:302-309,
    :311-317).  Returns ``pos [NW, H]`` (clamped into range) and ``inside [NW, H]``.
    """
    ctx = (window_keys - window_queries) // 2
    start = torch.arange(num_windows) * window_queries - ctx
    pos = start[:, None] + torch.arange(window_keys)[None, :]
    inside = (pos >= 0) & (pos < num_windows * window_queries)
    return pos.clamp(0, num_windows * window_queries - 1), inside


def attention_pair_bias_sliding_window(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    params: dict,
    num_heads: int,
    multiplicity: int = 1,
    initial_norm: bool = True,
    inf: float = 1e6,
) -> Tensor:
    """AttentionPairBiasSlidingWindow.forward (biomoa/ops/attention_pair_bias.py:277-340).

    s [B*M*NW, W, c_s], z [B, NW, W, H, c_z], mask [B*NW, W] bool -> [B*M*NW, W, c_s]
    (float32).  Rows of s are ordered (b, m, window); the keys of window w are
    the k/v rows of the same (b, m) sequence at ``sliding_window_keys`` (zero
    outside the sequence, :302-309), their mask is gathered the same way (False
    outside, :311-317); the pair bias ``proj_z(norm_z(z))`` is per (b, window)
    and shared by the M copies (:319, :328-330); masked keys are replaced by
    -inf (:332-334); out = proj_o(g * o) (:339-340).
    """
    s = _f32(s)
    z = _f32(z)
    mask = mask.bool().cpu()
    assert s.ndim == 3 and z.ndim == 5 and mask.ndim == 2  # :288
    M = multiplicity
    B, NW, W, H = z.shape[:4]
    folded, _, c_s = s.shape
    BM = folded // NW
    assert BM == B * M and s.shape[1] == W and mask.shape == (B * NW, W)
    nh = num_heads
    d = c_s // nh
    if initial_norm:
        s = _ln(s, params, "norm_s")  # :294-295
    wqkv = _p(params, "proj_qkv.weight")
    q = (s @ wqkv[:c_s].T + _p(params, "proj_q_bias")).view(BM, NW, W, nh, d)  # :297-299
    kvals = (s @ wqkv[c_s:2 * c_s].T).reshape(BM, NW * W, nh, d)
    vvals = (s @ wqkv[2 * c_s:].T).reshape(BM, NW * W, nh, d)
    g = torch.sigmoid(s @ _p(params, "proj_g.weight").T).view(BM, NW, W, c_s)  # :300
    pos, inside = sliding_window_keys(NW, W, H)
    kw = kvals[:, pos] * inside[None, :, :, None, None]  # [BM, NW, H, nh, d]
    vw = vvals[:, pos] * inside[None, :, :, None, None]
    key_ok = mask.view(B, NW * W)[:, pos] & inside[None]  # [B, NW, H]
    bias = (_ln(z, params, "norm_z") @ _p(params, "proj_z.weight").T).permute(0, 1, 4, 2, 3)  # [B,NW,nh,W,H] (:319)
    out = torch.empty(BM, NW, W, c_s)
    for bm in range(BM):
        b = bm // M
        logits = torch.einsum("wihd,wjhd->whij", q[bm], kw[bm]) / (d**0.5)  # :325-326
        logits = logits + bias[b]  # :328-330
        logits = logits.masked_fill(~key_ok[b][:, None, None, :], -inf)  # :332-334
        o = torch.einsum("whij,wjhd->wihd", logits.softmax(dim=-1), vw[bm])  # :336-337
        out[bm] = (g[bm] * o.reshape(NW, W, c_s)) @ _p(params, "proj_o.weight").T  # :339-340
    return out.view(folded, W, c_s)


# ----------------------------------------------------------------------------
# Pair glue either side of the trunk
# ----------------------------------------------------------------------------
def distogram(z: Tensor, params: dict) -> Tensor:
    """DistogramModule.forward (biomoa/modules/embedders.py:191-206): Linear(z + z^T), with bias.

    z [B,N,N,c_z] -> [B,N,N,num_bins] (float32); params ``distogram.{weight,bias}``.
    """
    z = _f32(z)
    sym = z + z.transpose(1, 2)  # :205
    return sym @ _p(params, "distogram.weight").T + _p(params, "distogram.bias")  # :206


def pairwise_conditioning(z_trunk: Tensor, rel_pos: Tensor, params: dict, num_transitions: int = 2) -> Tensor:
    """PairwiseConditioning.forward (biomoa/modules/diffusion.py:509-535).

    cat([z_trunk, rel_pos], -1) -> LayerNorm -> LinearNoBias (``dim_pairwise_init_proj``,
    :521-524), then ``z = transition(z) + z`` for each of ``transitions`` (:526-527).
    """
    x = torch.cat([_f32(z_trunk), _f32(rel_pos)], dim=-1)  # :521-523
    x = _ln(x, params, "dim_pairwise_init_proj.0") @ _p(params, "dim_pairwise_init_proj.1.weight").T  # :524
    for k in range(num_transitions):
        x = transition(x, _sub(params, f"transitions.{k}")) + x  # :526-527
    return x


# ----------------------------------------------------------------------------
# Outer product mean
# ----------------------------------------------------------------------------
def outer_product_mean(
    m: Tensor, mask: Tensor, params: dict, i_chunk: int | None = None, i_stop: int | None = None
) -> Tensor:
    """OuterProductMeanVanilla.forward (biomoa/ops/outer_product_mean.py:45-75).

    m [B,S,N,C_in], mask [B,S,N] or [B,N] -> [B,N,N,C_out] (float32).
    ``num_valid = mask.any(-1).sum(1).clamp(min=1)`` per batch for a [B,S,N]
    mask, 1 for a [B,N] mask (:67-70); flatten order c*C_H + d (:72-73); the
    mean is taken before the output projection (:74-75 and the memory-saving
    kernel's "normalize before the cast", ops/triton/opm.py:114-116).
    ``i_stop`` computes only output rows [0, i_stop) (rows beyond stay
    uninitialised; used to time a bounded sample).
    """
    m = _f32(m)
    mask = mask.bool().cpu()
    mp = _ln(m, params, "norm") @ _p(params, "proj_ab.weight").T  # :61
    mp = mp.masked_fill(~mask.unsqueeze(-1), 0.0)  # :62
    a, b = mp.chunk(2, dim=-1)  # :63
    if mask.ndim == 3:
        num_valid = mask.any(dim=-1).sum(dim=1).clamp(min=1).float()  # :68
    else:
        num_valid = torch.ones(m.shape[0])  # :70
    B, S, N, C = a.shape
    wo = _p(params, "proj_o.weight")
    bo = _p(params, "proj_o.bias")
    out = torch.empty(B, N, N, wo.shape[0])
    step = i_chunk or N
    for i0 in range(0, min(N, i_stop or N), step):
        i1 = min(N, i0 + step)
        zc = torch.einsum("bsic,bsjd->bijcd", a[:, :, i0:i1], b)  # :72
        zc = zc.reshape(B, i1 - i0, N, C * C)  # :73
        zc = zc / num_valid[:, None, None, None]  # :74
        out[:, i0:i1] = zc @ wo.T + bo  # :75
    return out


# ----------------------------------------------------------------------------
# Pair-weighted averaging (MSA module)
# ----------------------------------------------------------------------------
def pair_weighted_averaging(
    m: Tensor, z: Tensor, mask: Tensor, params: dict, num_heads: int = 8, c_h: int = 32, inf: float = 1e6
) -> Tensor:
    """PairWeightedAveraging.forward, unchunked path (biomoa/ops/pair_weighted_averaging.py:125-153).

    m [B,S,N,c_m], z [B,N,N,c_z], mask [B,N,N] -> [B,S,N,c_m] (float32).
    m' = LN_m(m) (:84); v = proj_m(m') split into heads (:127-129);
    b = proj_z(LN_z(z)) per head, masked_fill(~mask, -inf) (:131-143);
    w = softmax over j (:144); g = sigmoid(proj_g(m')) (:147-148);
    o[s,i,h] = sum_j w[h,i,j] v[s,j,h] with heads flattened h*c_h + d (:151-153);
    out = proj_o(g * o) (:154).  LN_z has a bias unless ``norm_z.bias`` is absent
    (use_bias_in_layer_norm=False, :134-141 -- the same values, computed fused).
    """
    m = _f32(m)
    z = _f32(z)
    mask = mask.bool().cpu()
    B, S, N, _ = m.shape
    mn = _ln(m, params, "norm_m")
    v = (mn @ _p(params, "proj_m.weight").T).reshape(B, S, N, num_heads, c_h).permute(0, 3, 1, 2, 4)
    b = (_ln(z, params, "norm_z") @ _p(params, "proj_z.weight").T).permute(0, 3, 1, 2)
    b = b.masked_fill(~mask[:, None], -inf)
    w = torch.softmax(b, dim=-1)
    g = torch.sigmoid(mn @ _p(params, "proj_g.weight").T)
    o = torch.einsum("bhij,bhsjd->bhsid", w, v)
    o = o.permute(0, 2, 3, 1, 4).reshape(B, S, N, num_heads * c_h)
    return (g * o) @ _p(params, "proj_o.weight").T


# ----------------------------------------------------------------------------
# Transition (SwiGLU MLP)
# ----------------------------------------------------------------------------
def transition(x: Tensor, params: dict, use_norm: bool = True) -> Tensor:
    """Transition.forward (biomoa/ops/transition.py:52-76): fc3(silu(fc1(xn)) * fc2(xn))."""
    x = _f32(x)
    if use_norm:
        x = _ln(x, params, "norm")  # :68-69
    a = F.silu(x @ _p(params, "fc1.weight").T)  # :71-72
    b = x @ _p(params, "fc2.weight").T  # :73
    return (a * b) @ _p(params, "fc3.weight").T  # :74-75


# ----------------------------------------------------------------------------
# Pairformer block (NOT in the reference: AF3 supplement Alg. 17 ordering)
# ----------------------------------------------------------------------------
def _sub(params: dict, prefix: str) -> dict:
    n = len(prefix) + 1
    return {k[n:]: v for k, v in params.items() if k.startswith(prefix + ".")}


def pairformer_block(
    s: Tensor,
    z: Tensor,
    token_mask: Tensor,
    params: dict,
    triatt_heads: int = 4,
    apb_heads: int = 16,
    triatt_row_chunk: int | None = None,
) -> tuple[Tensor, Tensor]:
    """One Pairformer block (AF3 suppl. Alg. 17) built from the reference ops.

    z += TriMulOut; z += TriMulIn; z += TriAttStart; z += TriAttEnd; z += Transition_z;
    s += APB(s, z, mask) (initial_norm=True); s += Transition_s.
    Residual form and dropout-at-eval identity follow PairMixerLayer.forward
    (biomoa/modules/pairmixer.py:446-456) and apply_axiswise_dropout
    (biomoa/ops/dropout.py:68-69).  pair_mask = mask_i & mask_j (pairmixer.py:263-264).
    """
    s = _f32(s)
    z = _f32(z)
    pm = pair_mask_from_token_mask(token_mask.cpu())
    z = z + trimul(z, pm, _sub(params, "tri_mul_out"), "outgoing")
    z = z + trimul(z, pm, _sub(params, "tri_mul_in"), "incoming")
    z = z + triangle_attention(
        z, pm, _sub(params, "tri_att_start"), triatt_heads, True, row_chunk=triatt_row_chunk
    )
    z = z + triangle_attention(
        z, pm, _sub(params, "tri_att_end"), triatt_heads, False, row_chunk=triatt_row_chunk
    )
    z = z + transition(z, _sub(params, "transition_z"))
    s = s + attention_pair_bias(
        s, z, token_mask.bool(), _sub(params, "attention_pair_bias"), apb_heads, tile_size=None
    )
    s = s + transition(s, _sub(params, "transition_s"))
    return s, z


# ----------------------------------------------------------------------------
# The reference trunk's layers (PairMixer)
# ----------------------------------------------------------------------------
def pairmixer_layer(s: Tensor, z: Tensor, pair_mask: Tensor, params: dict) -> tuple[Tensor, Tensor]:
    """PairMixerLayer.forward (biomoa/modules/pairmixer.py:430-456), eval mode.

    z += TriMulOut(z, pm); z += TriMulIn(z, pm); z += Transition_z(z); s passes
    through.  Dropout is the identity at eval (biomoa/ops/dropout.py:68-69).
    """
    s = _f32(s)
    z = _f32(z)
    pm = pair_mask.bool().cpu()
    z = z + trimul(z, pm, _sub(params, "tri_mul_out"), "outgoing")  # :447-449
    z = z + trimul(z, pm, _sub(params, "tri_mul_in"), "incoming")  # :450-452
    z = z + transition(z, _sub(params, "transition_z"))  # :454
    return s, z


def pairmixer_msa_layer(
    s: Tensor, z: Tensor, m: Tensor, token_mask: Tensor, msa_mask: Tensor, params: dict
) -> tuple[Tensor, Tensor, Tensor]:
    """PairMixerMSALayer.forward (biomoa/modules/pairmixer.py:711-757), eval mode.

    ``token_mask`` is the pair mask [B,T,T] (built as mask_i & mask_j,
    pairmixer.py:589).  m += PWA(m, z, token_mask); m += Transition_m(m);
    z += OPM(m, msa_mask); z += TriMulOut; z += TriMulIn; z += Transition_z.
    """
    s = None if s is None else _f32(s)  # s may be None (the MSA module runs with s=None, :284-294)
    z = _f32(z)
    m = _f32(m)
    pm = token_mask.bool().cpu()
    m = m + pair_weighted_averaging(m, z, pm, _sub(params, "pair_weighted_averaging"))  # :737-741
    m = m + transition(m, _sub(params, "msa_transition"))  # :742
    z = z + outer_product_mean(m, msa_mask, _sub(params, "outer_product_mean"))  # :745
    z = z + trimul(z, pm, _sub(params, "tri_mul_out"), "outgoing")  # :748-750
    z = z + trimul(z, pm, _sub(params, "tri_mul_in"), "incoming")  # :751-753
    z = z + transition(z, _sub(params, "z_transition"))  # :755
    return s, z, m


# ----------------------------------------------------------------------------
# PairMixer trunk above the layers
# ----------------------------------------------------------------------------
def ln_linear(x: Tensor, base: Tensor, params: dict, norm: str, linear: str) -> Tensor:
    """``base + linear(norm(x))`` with LayerNorm (affine) and a bias-free Linear: the recycling updates
    ``s = s_init + s_recycle(s_norm(s))`` and ``z = z_init + z_recycle(z_norm(z))``
    (biomoa/modules/pairmixer.py:281-282; layers at :186-191)."""
    x = _f32(x)
    return _f32(base) + _ln(x, params, norm) @ _p(params, linear + ".weight").T


def msa_embed(
    msa: Tensor,
    has_deletion: Tensor,
    deletion_value: Tensor,
    msa_paired: Tensor | None,
    emb: Tensor,
    params: dict,
) -> Tensor:
    """PairMixerMSAModule input projections (pairmixer.py:591-599):
    m = msa_proj(cat(msa, has_deletion, deletion_value[, msa_paired])) + s_proj(emb)[:, None]."""
    feats = [_f32(msa), _f32(has_deletion)[..., None], _f32(deletion_value)[..., None]]
    if msa_paired is not None:
        feats.append(_f32(msa_paired)[..., None])
    m = torch.cat(feats, dim=-1) @ _p(params, "msa_proj.weight").T  # :591-598
    return m + (_f32(emb) @ _p(params, "s_proj.weight").T).unsqueeze(1)  # :599


def pairmixer_module(s: Tensor, z: Tensor, pair_mask: Tensor, params: dict, num_blocks: int) -> tuple[Tensor, Tensor]:
    """PairMixerModule.forward (pairmixer.py:352-370): the layers in order, ``layers.{i}.*``."""
    for i in range(num_blocks):
        s, z = pairmixer_layer(s, z, pair_mask, _sub(params, f"layers.{i}"))
    return _f32(s), _f32(z)


def pairmixer_msa_module(
    z: Tensor,
    emb: Tensor,
    feats: dict,
    token_pad_mask: Tensor,
    params: dict,
    msa_blocks: int,
) -> Tensor:
    """PairMixerMSAModule.forward (pairmixer.py:553-611) with ``s=None``: embed the MSA, then run the MSA
    layers (``layers.{i}.*``, :602-610) with the pair mask mask_i & mask_j (:589); returns z."""
    m = msa_embed(feats["msa"], feats["has_deletion"], feats["deletion_value"], feats.get("msa_paired"), emb, params)
    pm = pair_mask_from_token_mask(token_pad_mask.cpu())
    z = _f32(z)
    for i in range(msa_blocks):
        _, z, m = pairmixer_msa_layer(None, z, m, pm, feats["msa_mask"], _sub(params, f"layers.{i}"))
    return z


def pairmixer_uncond(s_init: Tensor, z_init: Tensor, params: dict) -> tuple[Tensor, Tensor]:
    """The unconditional branch of PairMixerSequenceEmbedder.forward (pairmixer.py:266-273): s = s_init and
    z = z_init + uncond_transition(z_norm(z_init)), the transition being Transition(token_z, 4 token_z) with its
    own LayerNorm (:194-200; transition.py:52-91)."""
    s_init, z_init = _f32(s_init), _f32(z_init)
    zn = _ln(z_init, params, "z_norm")  # :272
    return s_init, z_init + transition(zn, _sub(params, "uncond_transition"))


def pairmixer_trunk(
    s_init: Tensor,
    z_init: Tensor,
    s_inputs: Tensor,
    feats: dict,
    params: dict,
    num_blocks: int,
    msa_blocks: int,
    num_steps_recycle: int = 0,
) -> tuple[Tensor, Tensor]:
    """The recycling loop of PairMixerSequenceEmbedder.forward (pairmixer.py:275-296) from the initial
    embeddings on: s and z start at zero (:257-258); each pass recycles them (``s_norm``/``s_recycle``,
    ``z_norm``/``z_recycle``), runs ``msa_module`` (s = None) and then ``pairmixer_module``."""
    s_init, z_init = _f32(s_init), _f32(z_init)
    s, z = torch.zeros_like(s_init), torch.zeros_like(z_init)  # :257-258
    pm = pair_mask_from_token_mask(feats["token_pad_mask"].cpu())  # :263-264
    for _ in range(num_steps_recycle + 1):
        s = ln_linear(s, s_init, params, "s_norm", "s_recycle")  # :281
        z = ln_linear(z, z_init, params, "z_norm", "z_recycle")  # :282
        z = pairmixer_msa_module(z, s_inputs, feats, feats["token_pad_mask"], _sub(params, "msa_module"),
                                 msa_blocks)  # :284-294
        s, z = pairmixer_module(s, z, pm, _sub(params, "pairmixer_module"), num_blocks)  # :296
    return s, z
