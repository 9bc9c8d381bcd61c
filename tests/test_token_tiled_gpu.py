"""Attention token side at the denoiser's shapes, where the output projection runs on the LDS-tiled 256 x 256
kernel (M rows x c_s >= 2M outputs; smaller token counts take the per-block GEMM, covered by the other APB / SWA
tests): AttentionPairBias with multiplicity 8 at N = 768 and the sliding-window attention at 6144 atoms x 8 copies,
against the fp32 oracle, including the fused residual and the int8-tail residual epilogues of that path."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.attention_pair_bias import AttentionPairBias
from bioemu2_amd.residual import join_stream, split_stream
from bioemu2_amd.workloads import init_module
from tests._helpers import max_abs, rel_l2, state
from tests.test_apb_transition_gpu import _apb, _apb_inputs
from tests.test_swa_gpu import _inputs as _swa_inputs
from tests.test_swa_gpu import _module as _swa_module

pytestmark = pytest.mark.gpu


def _check(got, want, tag):
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}", flush=True)
    assert err <= 2e-2 and rl2 <= 1e-2, (tag, err, rl2)


def test_apb_denoiser_shape(gpu_device):
    """B = 1, M = 8 copies, N = 768 with 76 masked keys: 6144 x 384 outputs (tiled output projection)."""
    m = _apb(gpu_device, initial_norm=False)
    s, z, mask = _apb_inputs(1, 768, gpu_device, mult=8, pad_keys=76)
    with torch.no_grad():
        got = m(s, z, mask, multiplicity=8).float().cpu()
    for bm in (0, 7):   # every copy is an independent attention over the same z and mask
        want = oracle.attention_pair_bias(s[bm:bm + 1].cpu(), z.cpu(), mask.cpu(), state(m), 16, initial_norm=False)
        _check(got[bm:bm + 1], want, f"apb denoiser copy {bm}")


def test_apb_denoiser_shape_residual_tail(gpu_device):
    """The same shape with the residual stream carried as bf16 + int8 tail, updated in place."""
    mod = init_module(AttentionPairBias(384, 128, 16, initial_norm=False), 5).to(gpu_device)
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(8, 768, 384, generator=g) * 3.0).to(gpu_device)
    z = torch.randn(1, 768, 768, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    mask = torch.ones(1, 768, dtype=torch.bool)
    mask[0, -76:] = False
    mk = _ops.mask_u8(mask.to(gpu_device))
    hi, tail = split_stream(x)
    seen = hi.float().cpu()
    _ops.launch_apb(hi, z, mk, *mod.prepared_params(), hi, 16, multiplicity=8, residual=True, tail=tail)
    got = join_stream(hi, tail).cpu()
    for bm in (0, 5):   # the op reads hi (its LayerNorm input); the residual it adds to is hi + tail ~ x
        want = x[bm:bm + 1].cpu() + oracle.attention_pair_bias(seen[bm:bm + 1], z.cpu(), mask, state(mod), 16,
                                                               initial_norm=False)
        _check(got[bm:bm + 1], want, f"apb tail copy {bm}")


def test_swa_denoiser_shape(gpu_device):
    """6144 atoms (192 windows) x 8 copies, 40 padded atoms: 49152 x 128 outputs (tiled output projection)."""
    mod = _swa_module(gpu_device, initial_norm=False)
    s, z, mask = _swa_inputs(1, 8, 192, 128, 128, 16, gpu_device, pad=40)
    with torch.no_grad():
        got = mod(s, z, mask, multiplicity=8).float().cpu()
    want = oracle.attention_pair_bias_sliding_window(s.cpu(), z.cpu(), mask.cpu(), state(mod), 4, multiplicity=8,
                                                     initial_norm=False)
    _check(got, want, "swa 6144 atoms x 8")


def test_swa_denoiser_shape_residual(gpu_device):
    """Fused residual (out = s + update, in place) on the tiled path equals the separate sum."""
    mod = _swa_module(gpu_device, initial_norm=False)
    s, z, mask = _swa_inputs(1, 8, 192, 128, 128, 16, gpu_device, pad=40, seed=3)
    P = mod.prepared_params()
    with torch.no_grad():
        upd = mod(s, z, mask, multiplicity=8)
        res = s.clone()
        _ops.launch_swa(res, z, _ops.mask_u8(mask), *P, res, 4, multiplicity=8, residual=True)
    want = s.float() + upd.float()
    assert max_abs(res.float().cpu(), want.cpu()) <= 2 ** -7 * (want.abs().max().item() + 1)


def test_swa_denoiser_shape_narrow(gpu_device):
    """c_s = 64 (2 heads) at 6144 atoms x 8 copies: 49152 x 64 outputs take the tiled output projection with fewer
    output columns than half a tile, whose columns past the 64 weight rows must read as zero, not past the weight."""
    print("swa narrow: c_s=64 heads=2 atoms=6144 M=8", flush=True)
    mod = _swa_module(gpu_device, c_s=64, c_z=16, heads=2, initial_norm=False)
    s, z, mask = _swa_inputs(1, 8, 192, 128, 64, 16, gpu_device, pad=40, seed=5)
    with torch.no_grad():
        got = mod(s, z, mask, multiplicity=8).float().cpu()
    want = oracle.attention_pair_bias_sliding_window(s.cpu(), z.cpu(), mask.cpu(), state(mod), 2, multiplicity=8,
                                                     initial_norm=False)
    _check(got, want, "swa 6144 atoms x 8, c_s 64")
