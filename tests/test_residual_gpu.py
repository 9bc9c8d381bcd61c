"""Residual tails on the GPU: split / join bit-exact against the numpy statement of the format, and every
op's tail epilogue (residual=1 with an int8 tail) against x + the fp32 oracle update.
Modules use the block's recipe (default init, zero parameters re-drawn N(0, 0.02)).

For an op with a tail the stream value x (fp32, not bf16-representable) is split into (hi, tail); the op
normalises hi (the bf16 stream) and adds its update to hi + tail, so the expected result is
x + update(hi) and the bound is north_star's bf16 bound on that sum.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.attention_pair_bias import AttentionPairBias
from bioemu2_amd.outer_product_mean import REGISTRY as OPM_REGISTRY
from bioemu2_amd.pair_weighted_averaging import PairWeightedAveraging
from bioemu2_amd.residual import join_stream, split_stream
from bioemu2_amd.strategy import make
from bioemu2_amd.transition import Transition
from bioemu2_amd.triangle_attention import REGISTRY as TRIATT_REGISTRY
from bioemu2_amd.triangle_multiplication import TriangleMultiplicationHip
from bioemu2_amd.workloads import init_module
from tests._helpers import max_abs, np_tail_decode, np_tail_encode, rel_l2, state

pytestmark = pytest.mark.gpu


def _stream(shape, device, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    return x.to(device)


def _check(got, want, tag):
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.2f}", flush=True)
    assert err <= 2e-2 and rl2 <= 1e-2, (tag, err, rl2)


def test_split_join_bit_exact(gpu_device):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-30, 30, 1 << 16))).astype(np.float32)
    hi, tail = _ops.stream_split(torch.from_numpy(x).to(gpu_device))
    want_hi, want_t = np_tail_encode(x)
    assert np.array_equal(hi.view(torch.int16).cpu().numpy().view(np.uint16), want_hi)
    assert np.array_equal(tail.cpu().numpy(), want_t)
    back = _ops.stream_join(hi, tail).cpu().numpy()
    assert np.array_equal(back.view(np.uint32), np_tail_decode(want_hi, want_t).view(np.uint32))


def test_join_to_bf16_is_hi(gpu_device):
    """A bf16 join returns hi, which equals the fp32 join rounded to bf16, on a stream an op has updated."""
    x = _stream((2, 40, 40, 128), gpu_device, 11, scale=3.0)
    hi, tail = split_stream(x)
    m = init_module(Transition(128, 512), 0).to(gpu_device)
    _ops.launch_transition_pair(hi, *m.prepared_params(), hi, residual=True, tail=tail)
    want = _ops.stream_join(hi, tail).to(torch.bfloat16)
    got = join_stream(hi, tail, torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def _run_with_tail(launch, x32):
    """launch(hi, tail) updates (hi, tail) in place; returns the joined fp32 result and hi as the op saw it."""
    hi, tail = split_stream(x32)
    seen = hi.float().cpu()
    launch(hi, tail)
    return join_stream(hi, tail).cpu(), seen


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_tail(gpu_device, outgoing):
    torch.manual_seed(1)
    mod = init_module(TriangleMultiplicationHip(128, "outgoing" if outgoing else "incoming"), 3)
    mod = mod.to(gpu_device)
    n = 70
    x = _stream((1, n, n, 128), gpu_device, 0, 3.0)
    pm = torch.rand(1, n, n, generator=torch.Generator().manual_seed(1)) > 0.2
    mk = _ops.mask_u8(pm.to(gpu_device))
    got, seen = _run_with_tail(
        lambda hi, t: _ops.launch_trimul(hi, mk, *mod.prepared_params(), hi, outgoing, residual=True, tail=t), x)
    want = x.cpu() + oracle.trimul(seen, pm, state(mod), "outgoing" if outgoing else "incoming")
    _check(got, want, f"trimul tail outgoing={outgoing}")


@pytest.mark.parametrize("starting", [True, False])
def test_triatt_tail(gpu_device, starting):
    torch.manual_seed(2)
    mod = init_module(make(TRIATT_REGISTRY, "hip", starting=starting, c_z=128, num_heads=4), 2).to(gpu_device)
    n = 90
    x = _stream((1, n, n, 128), gpu_device, 1, 3.0)
    pm = torch.rand(1, n, n, generator=torch.Generator().manual_seed(2)) > 0.2
    mk = _ops.mask_u8(pm.to(gpu_device))
    got, seen = _run_with_tail(
        lambda hi, t: _ops.launch_triatt(hi, mk, *mod.prepared_params(), hi, starting, residual=True, tail=t), x)
    want = x.cpu() + oracle.triangle_attention(seen, pm, state(mod), 4, starting)
    _check(got, want, f"triatt tail starting={starting}")


@pytest.mark.parametrize("dim", [128, 64])
def test_transition_rows_tail(gpu_device, dim):
    torch.manual_seed(3)
    mod = init_module(Transition(dim, 4 * dim), 4).to(gpu_device)
    x = _stream((3, 41, dim), gpu_device, 2, 3.0)
    got, seen = _run_with_tail(
        lambda hi, t: _ops.launch_transition_pair(hi, *mod.prepared_params(), hi, residual=True, tail=t), x)
    _check(got, x.cpu() + oracle.transition(seen, state(mod)), f"transition rows tail dim={dim}")


def test_transition_token_tail(gpu_device):
    torch.manual_seed(4)
    mod = init_module(Transition(384, 1536), 5).to(gpu_device)
    x = _stream((2, 50, 384), gpu_device, 3, 3.0)
    got, seen = _run_with_tail(
        lambda hi, t: _ops.launch_transition_token(hi, *mod.prepared_params(), hi, residual=True, tail=t), x)
    _check(got, x.cpu() + oracle.transition(seen, state(mod)), "transition token tail")


def test_apb_tail(gpu_device):
    torch.manual_seed(5)
    mod = init_module(AttentionPairBias(384, 128, 16, initial_norm=True), 5).to(gpu_device)
    n = 77
    x = _stream((2, n, 384), gpu_device, 4, 3.0)
    z = _stream((2, n, n, 128), gpu_device, 5).to(torch.bfloat16)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[1, -9:] = False
    mk = _ops.mask_u8(mask.to(gpu_device))
    got, seen = _run_with_tail(
        lambda hi, t: _ops.launch_apb(hi, z, mk, *mod.prepared_params(), hi, 16, residual=True, tail=t), x)
    want = x.cpu() + oracle.attention_pair_bias(seen, z.cpu(), mask, state(mod), 16, tile_size=None)
    _check(got, want, "apb tail")


def test_opm_tail(gpu_device):
    torch.manual_seed(6)
    mod = make(OPM_REGISTRY, "vanilla", c_in=64, c_hidden=32, c_out=128)
    with torch.no_grad():
        mod.proj_o.bias.normal_(0, 0.1)
    mod = mod.to(gpu_device)
    S, n = 24, 60
    m = _stream((1, S, n, 64), gpu_device, 6).to(torch.bfloat16)
    mask = torch.rand(1, S, generator=torch.Generator().manual_seed(3))[:, :, None].expand(1, S, n) > 0.2
    mask3, mean_rows = _ops.opm_mask3(mask.to(gpu_device), 1, S, n)
    x = _stream((1, n, n, 128), gpu_device, 7, 3.0)
    got, _ = _run_with_tail(
        lambda hi, t: _ops.launch_opm(m, mask3, mean_rows, *mod.prepared_params(), out=hi, z_res=hi, tail=t), x)
    _check(got, x.cpu() + oracle.outer_product_mean(m.cpu(), mask, state(mod)), "opm tail")


def test_pwa_tail(gpu_device):
    torch.manual_seed(7)
    mod = init_module(PairWeightedAveraging(c_m=64, c_z=128, c_h=32, num_heads=8), 7).to(gpu_device)
    S, n = 12, 64
    x = _stream((1, S, n, 64), gpu_device, 8, 3.0)
    z = _stream((1, n, n, 128), gpu_device, 9).to(torch.bfloat16)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, -5:] = False
    pm = tok[:, :, None] & tok[:, None, :]
    mk = _ops.mask_u8(pm.to(gpu_device))
    got, seen = _run_with_tail(
        lambda hi, t: _ops.launch_pwa(hi, z, mk, *mod.prepared_params(), hi, 8, residual=True, tail=t), x)
    want = x.cpu() + oracle.pair_weighted_averaging(seen, z.cpu(), pm, state(mod), num_heads=8, c_h=32)
    _check(got, want, "pwa tail")


def test_tail_without_residual_rejected(gpu_device):
    mod = Transition(128, 512).to(gpu_device)
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=gpu_device)
    t = torch.zeros(4, 128, dtype=torch.int8, device=gpu_device)
    with pytest.raises(ValueError):
        _ops.launch_transition_pair(x, *mod.prepared_params(), torch.empty_like(x), residual=False, tail=t)
