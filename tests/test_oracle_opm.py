"""Pins oracle.outer_product_mean (CPU) — follows biomoa/ops/outer_product_mean.py:45-75.

Pins: float64 brute force over S; masked rows contribute exact zeros
(test_outer_product_mean.py:286-310); the divisor is the per-batch count of
rows with any valid entry (duplicating the valid rows of the MSA leaves the
mean unchanged, doubling the divisor); flatten order c*C_H + d; a [B,N] mask
divides by 1.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from bioemu2_amd.outer_product_mean import OuterProductMeanHip
from tests._helpers import np_ln, np_params, randomize_params, state

CIN, CH, COUT = 12, 4, 10


def _params(seed=1):
    torch.manual_seed(seed)
    return state(randomize_params(OuterProductMeanHip(CIN, CH, COUT), seed))


def _inputs(B=2, S=5, N=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(B, S, N, CIN, generator=g)
    mask = torch.ones(B, S, N, dtype=torch.bool)
    mask[:, 1, -3:] = False  # test_outer_product_mean.py:102-114
    mask[0, -2:] = False
    return m, mask


def _brute(m, mask, P, mean_rows=True):
    P = np_params(P)
    mm = m.double().numpy()
    mk = mask.numpy()
    B, S, N, _ = mm.shape
    out = np.zeros((B, N, N, COUT))
    for b in range(B):
        a = np.zeros((S, N, CH))
        bb = np.zeros((S, N, CH))
        for s in range(S):
            for n in range(N):
                p = P["proj_ab.weight"] @ np_ln(mm[b, s, n], P["norm.weight"], P["norm.bias"])
                if mk[b, s, n]:
                    a[s, n], bb[s, n] = p[:CH], p[CH:]
        nv = max(1, int(mk[b].any(-1).sum())) if mean_rows else 1
        for i in range(N):
            for j in range(N):
                o = np.zeros((CH, CH))
                for s in range(S):
                    o += np.outer(a[s, i], bb[s, j])
                out[b, i, j] = P["proj_o.weight"] @ (o.reshape(-1) / nv) + P["proj_o.bias"]
    return out


def test_matches_brute_force():
    P = _params()
    m, mask = _inputs()
    got = oracle.outer_product_mean(m, mask, P)
    np.testing.assert_allclose(got.double().numpy(), _brute(m, mask, P), atol=1e-5, rtol=1e-4)


def test_flatten_order_is_c_major():
    """A transposed (d*C_H + c) flatten must disagree (guards the c*C_H + d order)."""
    P = _params()
    m, mask = _inputs()
    Q = dict(P)
    Q["proj_o.weight"] = P["proj_o.weight"].view(COUT, CH, CH).transpose(1, 2).reshape(COUT, CH * CH)
    assert (oracle.outer_product_mean(m, mask, P) - oracle.outer_product_mean(m, mask, Q)).abs().max() > 1e-3


def test_masked_rows_contribute_exact_zeros():
    P = _params()
    m, mask = _inputs()
    m2 = m.clone()
    m2[~mask] = 1000.0
    torch.testing.assert_close(oracle.outer_product_mean(m, mask, P), oracle.outer_product_mean(m2, mask, P),
                               atol=0, rtol=0)


def test_divisor_is_valid_row_count():
    """Appending copies of the valid rows doubles sum and divisor: the mean is unchanged."""
    P = _params()
    m, _ = _inputs(B=1)
    mask = torch.ones(1, 5, 4, dtype=torch.bool)
    mask[0, 3:] = False
    a = oracle.outer_product_mean(m, mask, P)
    m2 = torch.cat([m, m[:, :3]], 1)
    mask2 = torch.cat([mask, mask[:, :3]], 1)
    torch.testing.assert_close(oracle.outer_product_mean(m2, mask2, P), a, atol=1e-5, rtol=1e-5)


def test_2d_mask_divides_by_one():
    P = _params()
    m, _ = _inputs(B=1)
    tok = torch.tensor([[True, True, False, True]])
    got = oracle.outer_product_mean(m, tok, P)
    want = _brute(m, tok[:, None, :].expand(1, 5, 4), P, mean_rows=False)
    np.testing.assert_allclose(got.double().numpy(), want, atol=1e-5, rtol=1e-4)


def test_i_chunking_is_exact():
    P = _params()
    m, mask = _inputs(N=7)
    torch.testing.assert_close(oracle.outer_product_mean(m, mask, P), oracle.outer_product_mean(m, mask, P, i_chunk=3),
                               atol=0, rtol=0)
