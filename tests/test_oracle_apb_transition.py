"""Pins oracle.attention_pair_bias and oracle.transition (CPU).

APB follows biomoa/ops/attention_pair_bias.py:128-225; Transition follows
biomoa/ops/transition.py:52-76.  Pins: float64 brute force from the
definitions, reduction to torch SDPA, tiled == untiled, multiplicity ==
separate runs, bitwise padding invariance in f32 (test_attention_pair_bias.py:805-867).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from bioemu2_amd.attention_pair_bias import AttentionPairBias
from bioemu2_amd.transition import Transition
from tests._helpers import np_ln, np_params, np_sigmoid, randomize_params, state

CS, CZ, H = 32, 8, 4


def _apb_params(initial_norm=True, ln_bias=False, seed=5) -> dict:
    torch.manual_seed(seed)
    m = AttentionPairBias(CS, CZ, H, initial_norm=initial_norm, use_bias_in_layer_norm=ln_bias)
    return state(randomize_params(m, seed))


def _apb_inputs(B=2, n=6, mult=1, seed=0):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B * mult, n, CS, generator=g)
    z = torch.randn(B, n, n, CZ, generator=g)
    mask = torch.ones(B, n, dtype=torch.bool)
    mask[0, -2:] = False  # padded keys in batch 0 (test_attention_pair_bias.py:76-95 style)
    return s, z, mask


def _apb_brute(s, z, mask, P, initial_norm, mult=1):
    P = np_params(P)
    s = s.double().numpy()
    z = z.double().numpy()
    mask = mask.numpy()
    BM, n, cs = s.shape
    d = cs // H
    out = np.zeros_like(s)
    for bm in range(BM):
        b = bm // mult
        x = np.stack([np_ln(r, P["norm_s.weight"], P["norm_s.bias"]) for r in s[bm]]) if initial_norm else s[bm]
        qkv = x @ P["proj_qkv.weight"].T
        q, k, v = qkv[:, :cs] + P["proj_q_bias"], qkv[:, cs:2 * cs], qkv[:, 2 * cs:]
        g = np_sigmoid(x @ P["proj_g.weight"].T)
        o = np.zeros((n, cs))
        for h in range(H):
            sl = slice(h * d, (h + 1) * d)
            for i in range(n):
                logits = np.empty(n)
                for j in range(n):
                    if not mask[b, j]:
                        logits[j] = -1e6
                        continue
                    zn = np_ln(z[b, i, j], P["norm_z.weight"], P.get("norm_z.bias"))
                    logits[j] = q[i, sl] @ k[j, sl] / math.sqrt(d) + zn @ P["proj_z.weight"][h]
                w = np.exp(logits - logits.max())
                o[i, sl] = (w / w.sum()) @ v[:, sl]
        out[bm] = (g * o) @ P["proj_o.weight"].T
    return out


@pytest.mark.parametrize("initial_norm", [True, False])
def test_apb_matches_brute_force(initial_norm):
    P = _apb_params(initial_norm)
    s, z, mask = _apb_inputs()
    got = oracle.attention_pair_bias(s, z, mask, P, H, initial_norm=initial_norm)
    np.testing.assert_allclose(got.double().numpy(), _apb_brute(s, z, mask, P, initial_norm), atol=1e-5, rtol=1e-4)


def test_apb_layernorm_bias_variant():
    P = _apb_params(True, ln_bias=True)
    s, z, mask = _apb_inputs()
    got = oracle.attention_pair_bias(s, z, mask, P, H)
    np.testing.assert_allclose(got.double().numpy(), _apb_brute(s, z, mask, P, True), atol=1e-5, rtol=1e-4)


def test_apb_reduces_to_sdpa_with_additive_bias():
    P = _apb_params(False)
    s, z, _ = _apb_inputs()
    B, n = z.shape[:2]
    mask = torch.ones(B, n, dtype=torch.bool)
    got = oracle.attention_pair_bias(s, z, mask, P, H, initial_norm=False)
    d = CS // H
    qkv = s @ P["proj_qkv.weight"].T
    q, k, v = qkv.chunk(3, -1)
    q = (q + P["proj_q_bias"]).view(B, n, H, d).transpose(1, 2)
    k = k.view(B, n, H, d).transpose(1, 2)
    v = v.view(B, n, H, d).transpose(1, 2)
    bias = (F.layer_norm(z, (CZ,), P["norm_z.weight"]) @ P["proj_z.weight"].T).permute(0, 3, 1, 2)
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=bias).transpose(1, 2).reshape(B, n, CS)
    want = (torch.sigmoid(s @ P["proj_g.weight"].T) * o) @ P["proj_o.weight"].T
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_apb_tiled_equals_untiled():
    P = _apb_params()
    s, z, mask = _apb_inputs(n=9)
    a = oracle.attention_pair_bias(s, z, mask, P, H, tile_size=None)
    b = oracle.attention_pair_bias(s, z, mask, P, H, tile_size=4)
    torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)


def test_apb_multiplicity_equals_separate_runs():
    P = _apb_params()
    mult = 3
    s, z, mask = _apb_inputs(B=2, mult=mult)
    got = oracle.attention_pair_bias(s, z, mask, P, H, multiplicity=mult)
    for bm in range(2 * mult):
        b = bm // mult
        one = oracle.attention_pair_bias(s[bm:bm + 1], z[b:b + 1], mask[b:b + 1], P, H)
        torch.testing.assert_close(got[bm:bm + 1], one, atol=1e-6, rtol=1e-6)


def test_apb_padding_invariance_f32():
    """Appending masked tokens leaves valid outputs unchanged (test_attention_pair_bias.py:805-867)."""
    P = _apb_params()
    s, z, mask = _apb_inputs(B=1, n=7)
    pad = 5
    ps = torch.cat([s, torch.randn(1, pad, CS)], 1)
    pz = torch.randn(1, 7 + pad, 7 + pad, CZ)
    pz[:, :7, :7] = z
    pm = torch.cat([mask, torch.zeros(1, pad, dtype=torch.bool)], 1)
    a = oracle.attention_pair_bias(s, z, mask, P, H, tile_size=None)
    b = oracle.attention_pair_bias(ps, pz, pm, P, H, tile_size=None)[:, :7]
    # CPU GEMM blocking depends on N, so the oracle is invariant to 1 ulp-ish;
    # the HIP path is held to bit-exactness (tests/test_apb_gpu.py).
    torch.testing.assert_close(a, b, atol=1e-6, rtol=0)


def _tr_params(dim=16, hidden=64, use_norm=True, seed=9):
    torch.manual_seed(seed)
    return state(randomize_params(Transition(dim, hidden, use_norm=use_norm), seed))


@pytest.mark.parametrize("use_norm", [True, False])
def test_transition_matches_brute_force(use_norm):
    P = _tr_params(use_norm=use_norm)
    x = torch.randn(3, 5, 16)
    got = oracle.transition(x, P, use_norm=use_norm).double().numpy()
    Pn = np_params(P)
    want = np.zeros_like(got)
    for idx in np.ndindex(3, 5):
        v = x[idx].double().numpy()
        if use_norm:
            v = np_ln(v, Pn["norm.weight"], Pn["norm.bias"])
        a = Pn["fc1.weight"] @ v
        hid = a * np_sigmoid(a) * (Pn["fc2.weight"] @ v)
        want[idx] = Pn["fc3.weight"] @ hid
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-4)


def test_transition_swiglu_halves_are_not_symmetric():
    """Swapping fc1 and fc2 must change the result (silu applies to fc1 only)."""
    P = _tr_params()
    x = torch.randn(4, 16)
    Q = dict(P)
    Q["fc1.weight"], Q["fc2.weight"] = P["fc2.weight"], P["fc1.weight"]
    assert (oracle.transition(x, P) - oracle.transition(x, Q)).abs().max() > 1e-3
