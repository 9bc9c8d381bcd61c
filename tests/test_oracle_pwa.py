"""Pins oracle.pair_weighted_averaging (CPU) — follows biomoa/ops/pair_weighted_averaging.py:125-154.

Pins: float64 brute-force loops; a row whose keys are all masked averages v
uniformly over the N keys (masked_fill(-inf), not an additive bias); a row
with a single valid key returns that key's v exactly; the weights do not
depend on the MSA row (duplicating the MSA duplicates the output); an LN_z
without bias equals one with a zero bias.  A planted mistake (heads
flattened d*H + h instead of h*c_h + d) fails the brute force.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from bioemu2_amd.pair_weighted_averaging import PairWeightedAveraging
from tests._helpers import np_ln, np_params, np_sigmoid, randomize_params, state

CM, CZ, CH, H = 8, 6, 4, 2


def _params(seed=1, bias=True):
    torch.manual_seed(seed)
    return state(randomize_params(PairWeightedAveraging(CM, CZ, CH, H, use_bias_in_layer_norm=bias), seed))


def _inputs(B=2, S=3, N=5, seed=0):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(B, S, N, CM, generator=g)
    z = torch.randn(B, N, N, CZ, generator=g)
    tok = torch.ones(B, N, dtype=torch.bool)
    tok[-1, -2:] = False
    mask = tok[:, :, None] & tok[:, None, :]
    return m, z, mask


def _brute(m, z, mask, P, head_major=True):
    P = np_params(P)
    mm, zz, mk = m.double().numpy(), z.double().numpy(), mask.numpy()
    B, S, N, _ = mm.shape
    out = np.zeros((B, S, N, CM))
    for b in range(B):
        w = np.zeros((H, N, N))
        for h in range(H):
            for i in range(N):
                row = np.array([
                    P["proj_z.weight"][h] @ np_ln(zz[b, i, j], P["norm_z.weight"], P.get("norm_z.bias"))
                    if mk[b, i, j] else -1e6
                    for j in range(N)
                ])
                e = np.exp(row - row.max())
                w[h, i] = e / e.sum()
        for s in range(S):
            mn = [np_ln(mm[b, s, j], P["norm_m.weight"], P["norm_m.bias"]) for j in range(N)]
            v = np.stack([P["proj_m.weight"] @ x for x in mn])  # [N, H*CH]
            for i in range(N):
                o = np.zeros(H * CH)
                for h in range(H):
                    for d in range(CH):
                        acc = sum(w[h, i, j] * v[j, h * CH + d] for j in range(N))
                        o[h * CH + d if head_major else d * H + h] = acc
                g = np_sigmoid(P["proj_g.weight"] @ mn[i])
                out[b, s, i] = P["proj_o.weight"] @ (g * o)
    return out


def test_matches_brute_force():
    P = _params()
    m, z, mask = _inputs()
    got = oracle.pair_weighted_averaging(m, z, mask, P, num_heads=H, c_h=CH).double().numpy()
    np.testing.assert_allclose(got, _brute(m, z, mask, P), rtol=1e-4, atol=1e-5)


def test_planted_flatten_order_fails():
    P = _params()
    m, z, mask = _inputs()
    got = oracle.pair_weighted_averaging(m, z, mask, P, num_heads=H, c_h=CH).double().numpy()
    assert np.abs(got - _brute(m, z, mask, P, head_major=False)).max() > 1e-2


def test_fully_masked_row_is_uniform_average():
    P = _params()
    m, z, mask = _inputs(B=1, N=5)
    mask = torch.ones_like(mask)
    mask[0, 2, :] = False
    got = oracle.pair_weighted_averaging(m, z, mask, P, num_heads=H, c_h=CH).double()
    Pn = np_params(P)
    mm = m.double().numpy()
    for s in range(m.shape[1]):
        mn = np.stack([np_ln(mm[0, s, j], Pn["norm_m.weight"], Pn["norm_m.bias"]) for j in range(5)])
        v = mn @ Pn["proj_m.weight"].T
        g = np_sigmoid(Pn["proj_g.weight"] @ mn[2])
        want = Pn["proj_o.weight"] @ (g * v.mean(axis=0))
        np.testing.assert_allclose(got[0, s, 2].numpy(), want, rtol=1e-4, atol=1e-5)


def test_single_valid_key_selects_it():
    P = _params()
    m, z, mask = _inputs(B=1, N=5)
    mask = torch.zeros_like(mask)
    mask[0, 1, 3] = True
    got = oracle.pair_weighted_averaging(m, z, mask, P, num_heads=H, c_h=CH).double()
    Pn = np_params(P)
    mm = m.double().numpy()
    for s in range(m.shape[1]):
        mn = np.stack([np_ln(mm[0, s, j], Pn["norm_m.weight"], Pn["norm_m.bias"]) for j in range(5)])
        v3 = Pn["proj_m.weight"] @ mn[3]
        g = np_sigmoid(Pn["proj_g.weight"] @ mn[1])
        np.testing.assert_allclose(got[0, s, 1].numpy(), Pn["proj_o.weight"] @ (g * v3), rtol=1e-4, atol=1e-5)


def test_weights_independent_of_msa_row():
    P = _params()
    m, z, mask = _inputs(B=1, S=2)
    mm = torch.cat([m, m.flip(1)], dim=1)
    a = oracle.pair_weighted_averaging(m, z, mask, P, num_heads=H, c_h=CH)
    b = oracle.pair_weighted_averaging(mm, z, mask, P, num_heads=H, c_h=CH)
    torch.testing.assert_close(b[:, :2], a, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(b[:, 2:], a.flip(1), rtol=1e-6, atol=1e-6)


def test_ln_z_without_bias_equals_zero_bias():
    P = _params(bias=False)
    m, z, mask = _inputs()
    Pb = dict(P)
    Pb["norm_z.bias"] = torch.zeros(CZ)
    a = oracle.pair_weighted_averaging(m, z, mask, P, num_heads=H, c_h=CH)
    b = oracle.pair_weighted_averaging(m, z, mask, Pb, num_heads=H, c_h=CH)
    assert torch.equal(a, b)
