"""The reference trunk's PairMixer layers on the GPU vs the fp32 CPU oracle compositions.

The layers carry their residual streams (z, m) with int8 tails and return fp32
for fp32 inputs, so they are held to the bf16 bound itself (max-abs 2e-2,
rel-L2 1e-2) on every valid element.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd.pairmixer import PairMixerLayerHip, PairMixerMSALayerHip
from bioemu2_amd.workloads import init_module
from tests._helpers import max_abs, rel_l2, state

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("bf16_autocast")]


def _tok(B, n, n_pad, device):
    tok = torch.ones(B, n, dtype=torch.bool)
    if n_pad:
        tok[:, n - n_pad:] = False
    return tok.to(device)


def _check(name, got, want, sel):
    g, w = got.float().cpu()[sel], want[sel]
    err, rl2 = max_abs(g, w), rel_l2(g, w)
    print(f"{name}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={w.abs().max():.2f}", flush=True)
    assert err <= 2e-2 and rl2 <= 1e-2, (name, err, rl2)


def _randn(shape, g, device):
    """~N(0, 1), bf16-representable, held in fp32."""
    return torch.randn(*shape, generator=g).to(torch.bfloat16).float().to(device)


@pytest.mark.parametrize("n,n_pad", [(64, 0), (96, 9)])
def test_pairmixer_layer_matches_oracle(gpu_device, n, n_pad):
    torch.manual_seed(0)
    layer = init_module(PairMixerLayerHip(384, 128), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(1)
    s = _randn((1, n, 384), g, gpu_device)
    z = _randn((1, n, n, 128), g, gpu_device)
    tok = _tok(1, n, n_pad, gpu_device)
    pm = tok[:, :, None] & tok[:, None, :]
    s_got, z_got = layer(s, z, pm)
    assert s_got is s and z_got.dtype == torch.float32
    _, z_want = oracle.pairmixer_layer(s.cpu(), z.cpu(), pm.cpu(), state(layer))
    _check(f"pairmixer n={n}", z_got, z_want, pm.cpu())


@pytest.mark.parametrize("S,n,n_pad", [(16, 64, 0), (24, 80, 8)])
def test_pairmixer_msa_layer_matches_oracle(gpu_device, S, n, n_pad):
    torch.manual_seed(0)
    layer = init_module(PairMixerMSALayerHip(384, 64, 128, 0.15, 0.25), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(2)
    s = _randn((1, n, 384), g, gpu_device)
    z = _randn((1, n, n, 128), g, gpu_device)
    m = _randn((1, S, n, 64), g, gpu_device)
    tok = _tok(1, n, n_pad, gpu_device)
    pm = tok[:, :, None] & tok[:, None, :]
    msa_mask = tok[:, None, :].expand(1, S, n).clone()
    msa_mask[:, -3:] = False  # a few padded MSA rows
    _, z_got, m_got = layer(s, z, m, pm, msa_mask)
    _, z_want, m_want = oracle.pairmixer_msa_layer(s.cpu(), z.cpu(), m.cpu(), pm.cpu(), msa_mask.cpu(), state(layer))
    _check(f"pairmixer-msa S={S} n={n} m", m_got, m_want, tok.cpu()[:, None, :].expand(1, S, n))
    _check(f"pairmixer-msa S={S} n={n} z", z_got, z_want, pm.cpu())


def test_pairmixer_inplace_matches_out_of_place(gpu_device):
    torch.manual_seed(0)
    layer = init_module(PairMixerMSALayerHip(384, 64, 128, 0.15, 0.25), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(3)
    s = torch.randn(1, 48, 384, generator=g).to(torch.bfloat16).to(gpu_device)
    z = torch.randn(1, 48, 48, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    m = torch.randn(1, 8, 48, 64, generator=g).to(torch.bfloat16).to(gpu_device)
    tok = _tok(1, 48, 4, gpu_device)
    pm = tok[:, :, None] & tok[:, None, :]
    msa_mask = tok[:, None, :].expand(1, 8, 48).clone()
    from bioemu2_amd.residual import join_stream, split_stream

    _, z_new, m_new = layer(s, z, m, pm, msa_mask)
    (z2, zt), (m2, mt) = split_stream(z), split_stream(m)
    layer.forward_(s, z2, m2, pm, msa_mask, z_tail=zt, m_tail=mt)
    assert torch.equal(join_stream(z2, zt, torch.bfloat16), z_new)
    assert torch.equal(join_stream(m2, mt, torch.bfloat16), m_new)


def test_msa_mask_controls_pair_update(gpu_device):
    """As the reference's test_msa_mask_controls_pair_update (tests/biomoa/modules/test_pairmixer.py):
    changing a masked MSA row leaves z bit-identical; changing a valid row changes it."""
    torch.manual_seed(0)
    layer = init_module(PairMixerMSALayerHip(384, 64, 128, 0.0, 0.0), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(4)
    B, S, n = 1, 6, 40
    z = torch.randn(B, n, n, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    m = torch.randn(B, S, n, 64, generator=g).to(torch.bfloat16).to(gpu_device)
    pm = torch.ones(B, n, n, dtype=torch.bool, device=gpu_device)
    msa_mask = torch.ones(B, S, n, dtype=torch.bool, device=gpu_device)
    msa_mask[:, 4:] = False
    _, z_base, _ = layer(None, z, m, pm, msa_mask)
    m_masked = m.clone()
    m_masked[:, 5] += 10.0
    _, z_masked, _ = layer(None, z, m_masked, pm, msa_mask)
    m_valid = m.clone()
    m_valid[:, 0] += 10.0
    _, z_valid, _ = layer(None, z, m_valid, pm, msa_mask)
    assert torch.equal(z_masked, z_base)
    assert not torch.equal(z_valid, z_base)


def test_ragged_batch_equals_systems_alone(gpu_device):
    """As the reference's test_pairmixer_padding_integration: a ragged batch (short system padded to the
    long one's token and MSA-row counts) gives each system's valid outputs bit-identical to running it alone."""
    torch.manual_seed(0)
    layer = init_module(PairMixerMSALayerHip(384, 64, 128, 0.15, 0.25), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(6)
    sizes = [(37, 9), (70, 12)]  # (tokens, MSA rows)
    n_max, s_max = 70, 12
    z = torch.randn(2, n_max, n_max, 128, generator=g).to(torch.bfloat16)
    m = torch.randn(2, s_max, n_max, 64, generator=g).to(torch.bfloat16)
    tok = torch.zeros(2, n_max, dtype=torch.bool)
    msa_mask = torch.zeros(2, s_max, n_max, dtype=torch.bool)
    for b, (n, s) in enumerate(sizes):
        tok[b, :n] = True
        msa_mask[b, :s, :n] = True
    pm = tok[:, :, None] & tok[:, None, :]
    dev = gpu_device
    _, z_rag, m_rag = layer(None, z.to(dev), m.to(dev), pm.to(dev), msa_mask.to(dev))
    for b, (n, s) in enumerate(sizes):
        zb = z[b:b + 1, :n, :n].contiguous().to(dev)
        mb = m[b:b + 1, :s, :n].contiguous().to(dev)
        pmb = torch.ones(1, n, n, dtype=torch.bool, device=dev)
        mmb = torch.ones(1, s, n, dtype=torch.bool, device=dev)
        _, z_one, m_one = layer(None, zb, mb, pmb, mmb)
        dz = (z_rag[b, :n, :n].float() - z_one[0].float()).abs().max().item()
        dm = (m_rag[b, :s, :n].float() - m_one[0].float()).abs().max().item()
        print(f"system {b} (n={n}, S={s}): max |ragged - alone| z={dz:.3e} m={dm:.3e}")
        assert dz == 0.0 and dm == 0.0
