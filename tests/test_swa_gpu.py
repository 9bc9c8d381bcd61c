"""HIP sliding-window attention with pair bias vs the fp32 CPU oracle; exact masking, multiplicity, residual."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.attention_pair_bias import AttentionPairBiasSlidingWindow
from tests._helpers import max_abs, randomize_params, rel_l2, state

pytestmark = pytest.mark.gpu

ATOL = 2e-2
RTOL_L2 = 1e-2
W = 32


def _module(device, c_s=128, c_z=16, heads=4, H=128, initial_norm=True, ln_bias=False, seed=11):
    torch.manual_seed(seed)
    m = AttentionPairBiasSlidingWindow(c_s, c_z, heads, window_queries=W, window_keys=H,
                                       initial_norm=initial_norm, use_bias_in_layer_norm=ln_bias)
    return randomize_params(m, seed).to(device).eval()


def _inputs(B, M, NW, H, c_s, c_z, device, pad=0, seed=0):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B * M * NW, W, c_s, generator=g).to(torch.bfloat16)
    z = torch.randn(B, NW, W, H, c_z, generator=g).to(torch.bfloat16)
    mask = torch.ones(B, NW * W, dtype=torch.bool)
    if pad:
        mask[:, NW * W - pad:] = False
    if B > 1:
        mask[1, 5:9] = False   # a ragged hole in batch 1
    return s.to(device), z.to(device), mask.view(B * NW, W).to(device)


def _check(got, want, tag):
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize(
    "B,M,NW,H,c_s,heads,c_z,pad,initial_norm,ln_bias",
    [
        (1, 1, 4, 128, 128, 4, 16, 0, True, False),
        (2, 2, 5, 128, 128, 4, 16, 40, True, False),
        (1, 3, 3, 64, 64, 2, 32, 7, False, True),
        (1, 1, 2, 96, 384, 12, 16, 3, True, True),
        (1, 1, 1, 128, 128, 4, 16, 0, True, False),
    ],
)
def test_matches_oracle(gpu_device, B, M, NW, H, c_s, heads, c_z, pad, initial_norm, ln_bias):
    mod = _module(gpu_device, c_s, c_z, heads, H, initial_norm, ln_bias)
    s, z, mask = _inputs(B, M, NW, H, c_s, c_z, gpu_device, pad)
    with torch.no_grad():
        got = mod(s, z, mask, multiplicity=M).float().cpu()
    want = oracle.attention_pair_bias_sliding_window(s.cpu(), z.cpu(), mask.cpu(), state(mod), heads,
                                                     multiplicity=M, initial_norm=initial_norm)
    _check(got, want, f"swa B={B} M={M} NW={NW} H={H} c_s={c_s} c_z={c_z} pad={pad}")


def test_masked_atoms_do_not_leak(gpu_device):
    """Valid atoms' outputs are bit-identical when masked atoms' s change (they are only keys there)."""
    mod = _module(gpu_device)
    NW, pad = 6, 45
    s, z, mask = _inputs(1, 1, NW, 128, 128, 16, gpu_device, pad)
    s2 = s.clone()
    s2.view(NW * W, 128)[NW * W - pad:] = 3.0
    with torch.no_grad():
        a = mod(s, z, mask).view(NW * W, 128)[: NW * W - pad]
        b = mod(s2, z, mask).view(NW * W, 128)[: NW * W - pad]
    assert torch.equal(a, b)


def test_multiplicity_equals_separate_runs(gpu_device):
    mod = _module(gpu_device)
    B, M, NW = 2, 3, 4
    s, z, mask = _inputs(B, M, NW, 128, 128, 16, gpu_device, 10)
    with torch.no_grad():
        got = mod(s, z, mask, multiplicity=M).view(B, M, NW, W, 128)
        sv = s.view(B, M, NW, W, 128)
        for b in range(B):
            for m in range(M):
                one = mod(sv[b, m].contiguous(), z[b:b + 1].contiguous(), mask.view(B, NW, W)[b].contiguous())
                assert torch.equal(got[b, m], one)


def test_fused_residual(gpu_device):
    mod = _module(gpu_device)
    s, z, mask = _inputs(1, 2, 3, 128, 128, 16, gpu_device)
    P = mod.prepared_params()
    with torch.no_grad():
        upd = mod(s, z, mask, multiplicity=2)
        res = s.clone()
        _ops.launch_swa(res, z, _ops.mask_u8(mask), *P, res, 4, multiplicity=2, residual=True)
    want = s.float() + upd.float()
    assert max_abs(res.float().cpu(), want.cpu()) <= 2 ** -7 * (want.abs().max().item() + 1)


def test_rejects_unsupported_shapes(gpu_device):
    mod = _module(gpu_device, H=128)
    s, z, mask = _inputs(1, 1, 2, 128, 128, 16, gpu_device)
    with pytest.raises(ValueError):
        _ops.launch_swa(s, z[..., :100, :].contiguous(), _ops.mask_u8(mask), *mod.prepared_params(),
                        torch.empty_like(s), 4)
