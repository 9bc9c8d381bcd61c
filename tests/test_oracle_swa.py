"""Pins oracle.attention_pair_bias_sliding_window (CPU).

Follows biomoa/ops/attention_pair_bias.py:277-340.  Pins: a float64 brute
force over absolute atom positions; a planted one-hot pair bias that must
select the key the centred window puts at that slot (the window's own queries
sit at slots ctx .. ctx + W - 1); with H == W every window is an independent
full AttentionPairBias (the already pinned oracle.attention_pair_bias);
multiplicity == separate runs; keys past the sequence end behave exactly like
masked keys; a window whose keys are all masked averages v uniformly over its
H slots (padding slots carry v = 0).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from bioemu2_amd.attention_pair_bias import AttentionPairBiasSlidingWindow
from tests._helpers import np_ln, np_params, np_sigmoid, randomize_params, state

CS, CZ, NH = 16, 4, 2   # head dim 8
W = 4


def _params(H=8, initial_norm=True, ln_bias=False, seed=7) -> dict:
    torch.manual_seed(seed)
    m = AttentionPairBiasSlidingWindow(CS, CZ, NH, window_queries=W, window_keys=H, initial_norm=initial_norm,
                                       use_bias_in_layer_norm=ln_bias)
    return state(randomize_params(m, seed))


def _inputs(B=2, M=1, NW=3, H=8, seed=0, n_pad=(2, 0)):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B * M * NW, W, CS, generator=g)
    z = torch.randn(B, NW, W, H, CZ, generator=g)
    mask = torch.ones(B, NW * W, dtype=torch.bool)
    for b, p in enumerate(n_pad[:B]):
        if p:
            mask[b, -p:] = False
    return s, z, mask.view(B * NW, W)


def _brute(s, z, mask, P, M, initial_norm):
    """float64 loops: for each query atom p (window p // W) and each of the H key slots."""
    P = np_params(P)
    B, NW, _, H, _ = z.shape
    NA = NW * W
    ctx = (H - W) // 2
    d = CS // NH
    s = s.double().numpy().reshape(B, M, NA, CS)
    z = z.double().numpy()
    mask = mask.numpy().reshape(B, NA)
    out = np.zeros_like(s)
    for b in range(B):
        for m in range(M):
            x = s[b, m]
            if initial_norm:
                x = np.stack([np_ln(r, P["norm_s.weight"], P["norm_s.bias"]) for r in x])
            wq = P["proj_qkv.weight"]
            q = x @ wq[:CS].T + P["proj_q_bias"]
            k = x @ wq[CS:2 * CS].T
            v = x @ wq[2 * CS:].T
            gt = np_sigmoid(x @ P["proj_g.weight"].T)
            o = np.zeros((NA, CS))
            for p in range(NA):
                w, i = divmod(p, W)
                for h in range(NH):
                    sl = slice(h * d, (h + 1) * d)
                    logits = np.empty(H)
                    vals = np.zeros((H, d))
                    for t in range(H):
                        a = w * W + t - ctx          # atom at key slot t of window w
                        zn = np_ln(z[b, w, i, t], P["norm_z.weight"], P.get("norm_z.bias"))
                        if 0 <= a < NA and mask[b, a]:
                            logits[t] = q[p, sl] @ k[a, sl] / math.sqrt(d) + zn @ P["proj_z.weight"][h]
                        else:
                            logits[t] = -1e6
                        if 0 <= a < NA:
                            vals[t] = v[a, sl]
                    e = np.exp(logits - logits.max())
                    o[p, sl] = (e / e.sum()) @ vals
            out[b, m] = (gt * o) @ P["proj_o.weight"].T
    return out.reshape(B * M * NW, W, CS)


@pytest.mark.parametrize("initial_norm,ln_bias,M,H", [(True, False, 1, 8), (False, True, 2, 8), (True, True, 1, 12)])
def test_matches_brute_force(initial_norm, ln_bias, M, H):
    P = _params(H, initial_norm, ln_bias)
    s, z, mask = _inputs(M=M, H=H)
    got = oracle.attention_pair_bias_sliding_window(s, z, mask, P, NH, multiplicity=M, initial_norm=initial_norm)
    want = _brute(s, z, mask, P, M, initial_norm)
    np.testing.assert_allclose(got.numpy(), want, atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("shift", [0, W, -W])
def test_planted_bias_selects_the_centred_window_slot(shift):
    """With q.k = 0, v = s, g = 1/2 and a one-hot bias at slot ctx + i + shift, query i of window w
    returns half the position code of atom w W + i + shift: slot ctx + i is the query's own atom."""
    H, NW, B = 12, 4, 1
    ctx = (H - W) // 2
    NA = NW * W
    P = _params(H, initial_norm=False, ln_bias=False)
    P["proj_qkv.weight"] = torch.cat([torch.zeros(2 * CS, CS), torch.eye(CS)])
    P["proj_q_bias"] = torch.zeros(CS)
    P["proj_g.weight"] = torch.zeros(CS, CS)
    P["proj_o.weight"] = torch.eye(CS)
    P["norm_z.weight"] = torch.ones(CZ)
    P["proj_z.weight"] = torch.zeros(NH, CZ)
    P["proj_z.weight"][:, 0] = 15.0
    s = torch.zeros(NW, W, CS)
    s.view(NA, CS)[:, 0] = torch.arange(NA, dtype=torch.float32) + 1.0   # position code (never 0)
    z = torch.zeros(B, NW, W, H, CZ)
    z[..., 1] = 1.0                                                    # LN -> large negative channel 0
    z[..., 0] = -1.0
    rows = []
    for w in range(NW):
        for i in range(W):
            t = ctx + i + shift
            z[0, w, i, t, 0], z[0, w, i, t, 1] = 1.0, -1.0              # the one hot slot
            rows.append((w, i, w * W + i + shift))
    mask = torch.ones(B * NW, W, dtype=torch.bool)
    out = oracle.attention_pair_bias_sliding_window(s, z, mask, P, NH, initial_norm=False)
    for w, i, a in rows:
        if 0 <= a < NA:
            assert out[w, i, 0].item() == pytest.approx(0.5 * (a + 1.0), rel=1e-5)


def test_reduces_to_full_apb_per_window_when_h_equals_w():
    """H == W (no context): every window is an independent AttentionPairBias over its W atoms."""
    B, M, NW = 2, 2, 3
    P = _params(W)
    s, z, mask = _inputs(B=B, M=M, NW=NW, H=W)
    got = oracle.attention_pair_bias_sliding_window(s, z, mask, P, NH, multiplicity=M)
    # APB with batch b' = (b, w) and its M copies: rows ordered (b, w, m)
    s_apb = s.view(B, M, NW, W, CS).permute(0, 2, 1, 3, 4).reshape(B * NW * M, W, CS)
    want = oracle.attention_pair_bias(s_apb, z.reshape(B * NW, W, W, CZ), mask, P, NH, multiplicity=M)
    want = want.view(B, NW, M, W, CS).permute(0, 2, 1, 3, 4).reshape(B * M * NW, W, CS)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_multiplicity_equals_separate_runs():
    B, M, NW = 2, 3, 3
    P = _params()
    s, z, mask = _inputs(B=B, M=M, NW=NW)
    got = oracle.attention_pair_bias_sliding_window(s, z, mask, P, NH, multiplicity=M).view(B, M, NW, W, CS)
    sv = s.view(B, M, NW, W, CS)
    for b in range(B):
        for m in range(M):
            one = oracle.attention_pair_bias_sliding_window(
                sv[b, m], z[b:b + 1], mask.view(B, NW, W)[b], P, NH, multiplicity=1
            )
            torch.testing.assert_close(got[b, m], one, atol=1e-6, rtol=1e-6)


def test_keys_past_the_end_behave_like_masked_keys():
    """Appending a fully masked window leaves the original windows' outputs unchanged."""
    H, NW = 12, 3
    P = _params(H)
    s, z, mask = _inputs(B=1, NW=NW, H=H, n_pad=(0,))
    g = torch.Generator().manual_seed(9)
    s2 = torch.cat([s, torch.randn(1, W, CS, generator=g)])
    z2 = torch.cat([z, torch.randn(1, 1, W, H, CZ, generator=g)], dim=1)
    mask2 = torch.cat([mask, torch.zeros(1, W, dtype=torch.bool)])
    a = oracle.attention_pair_bias_sliding_window(s, z, mask, P, NH)
    b = oracle.attention_pair_bias_sliding_window(s2, z2, mask2, P, NH)[:NW]
    torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)


def test_all_masked_window_averages_uniformly_over_slots():
    """Every key of window 1 masked: each head's output is mean_t v(slot t), with v = 0 for padding slots."""
    H, NW = 8, 2
    ctx = (H - W) // 2
    P = _params(H, initial_norm=False)
    s, z, _ = _inputs(B=1, NW=NW, H=H, n_pad=(0,))
    mask = torch.zeros(NW, W, dtype=torch.bool)
    out = oracle.attention_pair_bias_sliding_window(s, z, mask, P, NH, initial_norm=False)
    x = s.view(NW * W, CS)
    v = x @ P["proj_qkv.weight"][2 * CS:].T
    g = torch.sigmoid(x @ P["proj_g.weight"].T)
    w = 1
    slots = [w * W + t - ctx for t in range(H)]
    vmean = sum(v[a] for a in slots if 0 <= a < NW * W) / H
    want = (g[w * W:(w + 1) * W] * vmean) @ P["proj_o.weight"].T
    torch.testing.assert_close(out[w], want, atol=1e-5, rtol=1e-5)
