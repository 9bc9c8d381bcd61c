"""HIP PairWeightedAveraging vs the fp32 CPU oracle; exact masking / padding invariance, fused residual."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.pair_weighted_averaging import PairWeightedAveraging
from tests._helpers import max_abs, randomize_params, rel_l2, state

pytestmark = pytest.mark.gpu

ATOL = 2e-2
RTOL_L2 = 1e-2


def _module(device, bias=True, seed=3) -> PairWeightedAveraging:
    torch.manual_seed(seed)
    m = randomize_params(PairWeightedAveraging(64, 128, 32, 8, use_bias_in_layer_norm=bias), seed)
    return m.to(device).eval()


def _inputs(B, S, N, device, n_pad=0, seed=0):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(B, S, N, 64, generator=g).to(torch.bfloat16)
    z = torch.randn(B, N, N, 128, generator=g).to(torch.bfloat16)
    tok = torch.ones(B, N, dtype=torch.bool)
    if n_pad:
        tok[:, N - n_pad:] = False
    mask = tok[:, :, None] & tok[:, None, :]
    return m.to(device), z.to(device), mask.to(device)


def _check(got, want, tag):
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("B,S,N,n_pad", [(1, 8, 64, 0), (2, 5, 50, 7), (1, 16, 300, 30), (1, 64, 256, 25)])
def test_matches_oracle(gpu_device, B, S, N, n_pad):
    mod = _module(gpu_device)
    m, z, mask = _inputs(B, S, N, gpu_device, n_pad)
    with torch.no_grad():
        got = mod(m, z, mask).float().cpu()
    want = oracle.pair_weighted_averaging(m.cpu(), z.cpu(), mask.cpu(), state(mod), num_heads=8, c_h=32)
    _check(got, want, f"pwa B={B} S={S} N={N} pad={n_pad}")


def test_ln_z_without_bias(gpu_device):
    mod = _module(gpu_device, bias=False)
    m, z, mask = _inputs(1, 8, 70, gpu_device, 5)
    with torch.no_grad():
        got = mod(m, z, mask).float().cpu()
    want = oracle.pair_weighted_averaging(m.cpu(), z.cpu(), mask.cpu(), state(mod), num_heads=8, c_h=32)
    _check(got, want, "pwa no LN_z bias")


def test_fully_masked_rows_and_ragged_mask(gpu_device):
    """A row with every key masked averages uniformly; an arbitrary (non-token) pair mask."""
    mod = _module(gpu_device)
    m, z, _ = _inputs(1, 8, 96, gpu_device)
    g = torch.Generator().manual_seed(5)
    mask = (torch.rand(1, 96, 96, generator=g) > 0.3).to(gpu_device)
    mask[0, 10, :] = False
    mask[0, 40, :] = False
    with torch.no_grad():
        got = mod(m, z, mask).float().cpu()
    want = oracle.pair_weighted_averaging(m.cpu(), z.cpu(), mask.cpu(), state(mod), num_heads=8, c_h=32)
    _check(got, want, "pwa ragged mask")


def test_masked_inputs_do_not_leak(gpu_device):
    """Valid outputs are bit-identical when masked tokens' m and masked pairs' z change."""
    mod = _module(gpu_device)
    N, pad = 80, 12
    m, z, mask = _inputs(1, 8, N, gpu_device, pad)
    m2, z2 = m.clone(), z.clone()
    m2[:, :, N - pad:] = 7.0
    z2[:, N - pad:] = -3.0
    z2[:, :, N - pad:] = 5.0
    with torch.no_grad():
        a = mod(m, z, mask)[:, :, : N - pad]
        b = mod(m2, z2, mask)[:, :, : N - pad]
    assert torch.equal(a, b)


def test_fused_residual_and_determinism(gpu_device):
    mod = _module(gpu_device)
    m, z, mask = _inputs(1, 16, 128, gpu_device, 10)
    P = mod.prepared_params()
    mk = _ops.mask_u8(mask)
    with torch.no_grad():
        upd = mod(m, z, mask)
        out = torch.empty_like(m)
        _ops.launch_pwa(m, z, mk, *P, out, 8)
        assert torch.equal(out, upd)
        res = m.clone()
        _ops.launch_pwa(res, z, mk, *P, res, 8, residual=True)
    want = (m.float() + upd.float()).to(torch.bfloat16)
    # one bf16 rounding of the sum either way
    assert max_abs(res.float().cpu(), want.float().cpu()) <= 2 ** -7 * (m.float().abs().max().item() + 1)


def test_msa_config3_shape(gpu_device):
    """MSA-module shape (S=1024, N=512, trailing padded tokens): every MSA row against the oracle."""
    mod = _module(gpu_device)
    m, z, mask = _inputs(1, 1024, 512, gpu_device, 51)
    with torch.no_grad():
        got = mod(m, z, mask).float().cpu()
    want = oracle.pair_weighted_averaging(m.cpu(), z.cpu(), mask.cpu(), state(mod), num_heads=8, c_h=32)
    _check(got, want, "pwa S=1024 N=512")
