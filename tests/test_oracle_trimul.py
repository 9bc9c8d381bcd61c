"""Pins oracle.trimul (CPU) against brute force, identities and reference invariances."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from bioemu2_amd.triangle_multiplication import TriangleMultiplicationHip
from tests._helpers import np_ln, np_params, np_sigmoid, redraw_zero_params, state


def _params(dim: int, seed: int = 42) -> dict:
    torch.manual_seed(seed)
    return state(redraw_zero_params(TriangleMultiplicationHip(dim=dim)))


def _inputs(n: int, dim: int, seed: int = 0):
    torch.manual_seed(seed)
    x = torch.randn(1, n, n, dim)
    mask = torch.rand(1, n, n) > 0.25  # test_triangle_multiplication.py:150-151
    return x, mask


def _brute(x: torch.Tensor, mask: torch.Tensor, params: dict, mode: str) -> np.ndarray:
    P = np_params(params)
    xx = x[0].double().numpy()
    mm = mask[0].numpy()
    n, _, d = xx.shape
    xn = np.zeros_like(xx)
    a = np.zeros_like(xx)
    b = np.zeros_like(xx)
    for i in range(n):
        for j in range(n):
            v = np_ln(xx[i, j], P["norm_in.weight"], P["norm_in.bias"])
            xn[i, j] = v
            pr = (P["p_in.weight"] @ v) * np_sigmoid(P["g_in.weight"] @ v)
            if not mm[i, j]:
                pr[:] = 0.0
            a[i, j] = pr[:d]
            b[i, j] = pr[d:]
    out = np.zeros_like(xx)
    for i in range(n):
        for j in range(n):
            o = np.zeros(d)
            for k in range(n):
                if mode == "outgoing":
                    o += a[i, k] * b[j, k]
                else:
                    o += a[k, i] * b[k, j]
            on = np_ln(o, P["norm_out.weight"], P["norm_out.bias"])
            out[i, j] = (P["p_out.weight"] @ on) * np_sigmoid(P["g_out.weight"] @ xn[i, j])
    return out


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_trimul_matches_brute_force(mode):
    params = _params(8)
    x, mask = _inputs(5, 8)
    got = oracle.trimul(x, mask, params, mode)[0].double().numpy()
    np.testing.assert_allclose(got, _brute(x, mask, params, mode), atol=2e-5, rtol=1e-4)


def test_incoming_is_outgoing_of_transpose_with_swapped_halves():
    """incoming(x) == outgoing(x^T, a<->b halves swapped)^T  (transposed-operand check)."""
    params = _params(16)
    x, mask = _inputs(9, 16)
    swapped = dict(params)
    d = 16
    for key in ("p_in.weight", "g_in.weight"):
        w = params[key]
        swapped[key] = torch.cat([w[d:], w[:d]], dim=0)
    inc = oracle.trimul(x, mask, params, "incoming")
    out_t = oracle.trimul(x.transpose(1, 2), mask.transpose(1, 2), swapped, "outgoing").transpose(1, 2)
    torch.testing.assert_close(inc, out_t, atol=2e-5, rtol=1e-5)
    # Without the swap the identity must fail (guards against a vacuous check).
    wrong = oracle.trimul(x.transpose(1, 2), mask.transpose(1, 2), params, "outgoing").transpose(1, 2)
    assert (wrong - inc).abs().max() > 1e-3


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_masking_bit_exact(mode):
    """test_triangle_multiplication.py:373-388: masked inputs do not change valid outputs."""
    params = _params(16)
    x, mask = _inputs(12, 16)
    changed = x.clone()
    changed[~mask] = 1000.0
    a = oracle.trimul(x, mask, params, mode)
    b = oracle.trimul(changed, mask, params, mode)
    torch.testing.assert_close(b[mask], a[mask], atol=0.0, rtol=0.0)


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_padding_invariance(mode):
    """test_triangle_multiplication.py:303-329 with 1000.0 padding (:163-170)."""
    params = _params(16)
    n, pad, d = 12, 4, 16
    x, mask = _inputs(n, d)
    px = x.new_full((1, n + pad, n + pad, d), 1000.0)
    px[:, :n, :n] = x
    pm = mask.new_zeros(1, n + pad, n + pad)
    pm[:, :n, :n] = mask
    a = oracle.trimul(x, mask, params, mode)
    b = oracle.trimul(px, pm, params, mode)[:, :n, :n]
    torch.testing.assert_close(b, a, atol=1e-6, rtol=0.0)


def test_all_masked_gives_closed_form():
    """mask == 0 everywhere => out = p_out(LN_out(0)) * sigmoid(g_out(LN_in(x)))."""
    params = _params(16)
    x, _ = _inputs(6, 16)
    mask = torch.zeros(1, 6, 6, dtype=torch.bool)
    got = oracle.trimul(x, mask, params, "outgoing")
    ln_out_zero = params["norm_out.bias"]  # LN of a zero vector = beta
    xn = torch.nn.functional.layer_norm(x, (16,), params["norm_in.weight"], params["norm_in.bias"])
    want = (ln_out_zero @ params["p_out.weight"].T) * torch.sigmoid(xn @ params["g_out.weight"].T)
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)
