"""Pins oracle.triangle_attention (CPU): brute force, identities and closed forms.

Triangle attention is not in the reference (biomoa/modules/pairmixer.py:459-462);
the oracle restates AF3 suppl. Alg. 14/15 with the reference's masked_fill(-1e6)
key masking (biomoa/ops/attention_pair_bias.py:184-190).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from bioemu2_amd.triangle_attention import TriangleAttentionHip
from tests._helpers import np_ln, np_params, np_sigmoid, randomize_params, state


def _params(c: int = 16, H: int = 4, seed: int = 3) -> dict:
    torch.manual_seed(seed)
    return state(randomize_params(TriangleAttentionHip(c_z=c, num_heads=H), seed))


def _inputs(n: int, c: int = 16, seed: int = 0, p_valid: float = 0.8):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, c, generator=g)
    mask = torch.rand(1, n, n, generator=g) < p_valid
    return z, mask


def _brute(z, mask, P, H, starting):
    """Triple loop in float64 straight from the algorithm's definition."""
    P = np_params(P)
    zz = z[0].double().numpy()
    mm = mask[0].numpy()
    if not starting:
        zz = zz.transpose(1, 0, 2)
        mm = mm.T
    n, _, c = zz.shape
    d = c // H
    zn = np.zeros_like(zz)
    for a in range(n):
        for b in range(n):
            zn[a, b] = np_ln(zz[a, b], P["norm.weight"], P["norm.bias"])
    q = zn @ P["proj_q.weight"].T
    k = zn @ P["proj_k.weight"].T
    v = zn @ P["proj_v.weight"].T
    g = np_sigmoid(zn @ P["proj_g.weight"].T)
    bias = zn @ P["proj_b.weight"].T  # [j, k, h]
    out = np.zeros_like(zz)
    for i in range(n):
        for j in range(n):
            o = np.zeros(c)
            for h in range(H):
                sl = slice(h * d, (h + 1) * d)
                logits = np.array(
                    [
                        (q[i, j, sl] @ k[i, kk, sl]) / math.sqrt(d) + bias[j, kk, h]
                        if mm[i, kk]
                        else -1e6
                        for kk in range(n)
                    ]
                )
                w = np.exp(logits - logits.max())
                w /= w.sum()
                o[sl] = w @ v[i, :, sl]
            out[i, j] = (g[i, j] * o) @ P["proj_o.weight"].T
    if not starting:
        out = out.transpose(1, 0, 2)
    return out


@pytest.mark.parametrize("starting", [True, False])
def test_matches_brute_force(starting):
    P = _params()
    z, mask = _inputs(6)
    got = oracle.triangle_attention(z, mask, P, 4, starting)[0].double().numpy()
    np.testing.assert_allclose(got, _brute(z, mask, P, 4, starting), atol=1e-5, rtol=1e-4)


def test_ending_is_starting_of_transpose():
    P = _params()
    z, mask = _inputs(9)
    end = oracle.triangle_attention(z, mask, P, 4, starting=False)
    st = oracle.triangle_attention(z.transpose(1, 2), mask.transpose(1, 2), P, 4, True).transpose(1, 2)
    torch.testing.assert_close(end, st, atol=1e-6, rtol=1e-6)
    # the two nodes differ on a non-symmetric input (the check is not vacuous)
    assert (oracle.triangle_attention(z, mask, P, 4, True) - end).abs().max() > 1e-3


def test_zero_bias_full_mask_reduces_to_sdpa():
    """proj_b = 0, all keys valid => per-row scaled-dot-product attention."""
    P = _params()
    P["proj_b.weight"] = torch.zeros_like(P["proj_b.weight"])
    n, c, H = 7, 16, 4
    d = c // H
    z, _ = _inputs(n)
    mask = torch.ones(1, n, n, dtype=torch.bool)
    got = oracle.triangle_attention(z, mask, P, H, True)
    zn = F.layer_norm(z, (c,), P["norm.weight"], P["norm.bias"])
    q = (zn @ P["proj_q.weight"].T).view(1, n, n, H, d).permute(0, 1, 3, 2, 4)  # [b,i,h,j,d]
    k = (zn @ P["proj_k.weight"].T).view(1, n, n, H, d).permute(0, 1, 3, 2, 4)
    v = (zn @ P["proj_v.weight"].T).view(1, n, n, H, d).permute(0, 1, 3, 2, 4)
    o = F.scaled_dot_product_attention(q, k, v).permute(0, 1, 3, 2, 4).reshape(1, n, n, c)
    want = (torch.sigmoid(zn @ P["proj_g.weight"].T) * o) @ P["proj_o.weight"].T
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_fully_masked_row_gives_uniform_average():
    """masked_fill(-1e6) on every key => uniform weights over all keys."""
    P = _params()
    n, c, H = 5, 16, 4
    z, mask = _inputs(n)
    mask[0, 2, :] = False
    got = oracle.triangle_attention(z, mask, P, H, True)[0, 2]
    zn = F.layer_norm(z, (c,), P["norm.weight"], P["norm.bias"])[0, 2]
    v = zn @ P["proj_v.weight"].T
    o = v.mean(0, keepdim=True).expand(n, c)
    want = (torch.sigmoid(zn @ P["proj_g.weight"].T) * o) @ P["proj_o.weight"].T
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_row_chunking_is_exact():
    P = _params()
    z, mask = _inputs(10)
    a = oracle.triangle_attention(z, mask, P, 4, True)
    b = oracle.triangle_attention(z, mask, P, 4, True, row_chunk=3)
    torch.testing.assert_close(a, b, atol=0, rtol=0)
