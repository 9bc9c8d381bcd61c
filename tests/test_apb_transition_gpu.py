"""HIP AttentionPairBias and Transition vs the fp32 CPU oracle; bit-exact padding invariance."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.attention_pair_bias import AttentionPairBias
from bioemu2_amd.transition import Transition
from tests._helpers import max_abs, randomize_params, rel_l2, state

pytestmark = pytest.mark.gpu

ATOL = 2e-2  # north_star bf16 tolerance vs the fp32 oracle
RTOL_L2 = 1e-2


def _apb(device, initial_norm=True, ln_bias=False, c_s=384, H=16, seed=11):
    torch.manual_seed(seed)
    m = AttentionPairBias(c_s, 128, H, initial_norm=initial_norm, use_bias_in_layer_norm=ln_bias)
    with torch.no_grad():
        m.proj_q_bias.normal_(0, 0.5)  # exercise the q bias (zero-initialised in the module)
    return m.to(device).eval()


def _apb_inputs(B, n, device, mult=1, pad_keys=0, c_s=384, seed=0):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B * mult, n, c_s, generator=g).to(torch.bfloat16)
    z = torch.randn(B, n, n, 128, generator=g).to(torch.bfloat16)
    mask = torch.ones(B, n, dtype=torch.bool)
    for b in range(B):  # test_attention_pair_bias.py:76-95: min((b+1)*3, n-4) padded keys
        k = pad_keys if pad_keys else min((b + 1) * 3, n - 4)
        mask[b, n - k:] = False
    return s.to(device), z.to(device), mask.to(device)


def _check(got, want, tag):
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("initial_norm", [True, False])
@pytest.mark.parametrize("n", [17, 64, 130])
def test_apb_matches_oracle(gpu_device, initial_norm, n):
    m = _apb(gpu_device, initial_norm)
    s, z, mask = _apb_inputs(2, n, gpu_device)
    with torch.no_grad():
        got = m(s, z, mask).float().cpu()
    want = oracle.attention_pair_bias(s.cpu(), z.cpu(), mask.cpu(), state(m), 16, initial_norm=initial_norm)
    _check(got, want, f"apb n={n} initial_norm={initial_norm}")


def test_apb_layernorm_bias(gpu_device):
    """norm_z with a bias (use_bias_in_layer_norm=True)."""
    m = _apb(gpu_device, True, ln_bias=True)
    with torch.no_grad():
        m.norm_z.bias.normal_(0, 0.3)
    s, z, mask = _apb_inputs(1, 50, gpu_device)
    with torch.no_grad():
        got = m(s, z, mask).float().cpu()
    want = oracle.attention_pair_bias(s.cpu(), z.cpu(), mask.cpu(), state(m), 16)
    _check(got, want, "apb ln-bias")


def test_apb_config2_shape(gpu_device):
    """Config 2: B=8, N=512, H=16 x 24, last 51 keys masked; every batch row against the oracle."""
    m = _apb(gpu_device)
    s, z, mask = _apb_inputs(8, 512, gpu_device, pad_keys=51)
    with torch.no_grad():
        got = m(s, z, mask).float().cpu()
    want = oracle.attention_pair_bias(s.cpu(), z.cpu(), mask.cpu(), state(m), 16)
    _check(got, want, "apb config2")


def test_apb_config5_shape(gpu_device):
    """The Pairformer block's attention at config 5's size: B=1, N=2048 with the last 102 keys masked."""
    m = _apb(gpu_device)
    s, z, mask = _apb_inputs(1, 2048, gpu_device, pad_keys=102, seed=5)
    with torch.no_grad():
        got = m(s, z, mask).float().cpu()
    want = oracle.attention_pair_bias(s.cpu(), z.cpu(), mask.cpu(), state(m), 16)
    _check(got, want, "apb n=2048")


def test_apb_multiplicity_equals_separate(gpu_device):
    m = _apb(gpu_device)
    mult = 3
    s, z, mask = _apb_inputs(2, 40, gpu_device, mult=mult)
    with torch.no_grad():
        both = m(s, z, mask, multiplicity=mult)
        for bm in range(2 * mult):
            b = bm // mult
            one = m(s[bm:bm + 1], z[b:b + 1], mask[b:b + 1])
            assert torch.equal(both[bm:bm + 1], one)


def test_apb_padding_bit_exact(gpu_device):
    m = _apb(gpu_device)
    n, pad = 45, 40
    s, z, mask = _apb_inputs(1, n, gpu_device)
    ps = torch.cat([s, torch.full((1, pad, 384), 7.0, dtype=s.dtype, device=gpu_device)], 1)
    pz = torch.full((1, n + pad, n + pad, 128), 1000.0, dtype=z.dtype, device=gpu_device)
    pz[:, :n, :n] = z
    pm = torch.cat([mask, torch.zeros(1, pad, dtype=torch.bool, device=gpu_device)], 1)
    with torch.no_grad():
        a = m(s, z, mask)
        b = m(ps, pz, pm)[:, :n]
    assert torch.equal(a, b)


def test_apb_masked_keys_bit_exact(gpu_device):
    """Values of s and z at masked keys never reach the outputs of valid tokens."""
    m = _apb(gpu_device)
    s, z, mask = _apb_inputs(2, 60, gpu_device)
    s2, z2 = s.clone(), z.clone()
    for b in range(2):
        s2[b, ~mask[b]] = 50.0
        z2[b][:, ~mask[b]] = 1000.0
    with torch.no_grad():
        a, b_ = m(s, z, mask), m(s2, z2, mask)
    assert torch.equal(a[mask], b_[mask])


def test_apb_fully_masked_row_is_uniform(gpu_device):
    m = _apb(gpu_device)
    s, z, mask = _apb_inputs(1, 33, gpu_device)
    mask[:] = False
    with torch.no_grad():
        got = m(s, z, mask).float().cpu()
    want = oracle.attention_pair_bias(s.cpu(), z.cpu(), mask.cpu(), state(m), 16)
    _check(got, want, "apb fully masked")


def test_apb_fused_residual(gpu_device):
    m = _apb(gpu_device)
    s, z, mask = _apb_inputs(1, 64, gpu_device)
    with torch.no_grad():
        upd = m(s, z, mask)
        ss = s.clone()
        _ops.launch_apb(ss, z, _ops.mask_u8(mask), *m.prepared_params(), ss, 16, residual=True)
    ref = s.float() + upd.float()
    assert max_abs(ss.float(), ref) <= 2 ** -7 * ref.abs().max().item()


def _transition(device, dim, hidden, use_norm=True, seed=4):
    torch.manual_seed(seed)
    return randomize_params(Transition(dim, hidden, use_norm=use_norm), seed).to(device).eval()


@pytest.mark.parametrize("use_norm", [True, False])
@pytest.mark.parametrize("n", [8, 45, 100])
def test_pair_transition_matches_oracle(gpu_device, use_norm, n):
    m = _transition(gpu_device, 128, 512, use_norm)
    x = torch.randn(1, n, n, 128).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        got = m(x).float().cpu()
    want = oracle.transition(x.cpu(), state(m), use_norm=use_norm)
    _check(got, want, f"pair transition n={n} use_norm={use_norm}")


@pytest.mark.parametrize("rows", [1, 37, 768])
def test_token_transition_matches_oracle(gpu_device, rows):
    m = _transition(gpu_device, 384, 1536)
    x = torch.randn(1, rows, 384).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        got = m(x).float().cpu()
    want = oracle.transition(x.cpu(), state(m))
    _check(got, want, f"token transition rows={rows}")


@pytest.mark.parametrize("use_norm", [True, False])
@pytest.mark.parametrize("shape", [(1, 7, 33), (2, 16, 64), (1, 1, 1)])
def test_msa_transition_matches_oracle(gpu_device, use_norm, shape):
    """The MSA representation's transition (dim 64, hidden 256) over [B,S,N,64] rows: the fused
    row kernel (ragged row counts, a single row) and, on the same input, the token LN + GEMM path."""
    m = _transition(gpu_device, 64, 256, use_norm)
    x = torch.randn(*shape, 64).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        got = m(x).float().cpu()
        tok = torch.empty_like(x)
        _ops.launch_transition_token(x, *m.prepared_params(), tok)
    want = oracle.transition(x.cpu(), state(m), use_norm=use_norm)
    _check(got, want, f"msa transition {shape} use_norm={use_norm}")
    _check(tok.float().cpu(), want, f"msa transition (token path) {shape} use_norm={use_norm}")


def test_msa_transition_residual_and_rowwise(gpu_device):
    m = _transition(gpu_device, 64, 256)
    x = torch.randn(1, 40, 70, 64).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        upd = m(x)
        assert torch.equal(m(x[:, 13:14]), upd[:, 13:14])
        xx = x.clone()
        _ops.launch_transition_pair(xx, *m.prepared_params(), xx, residual=True)
    ref = x.float() + upd.float()
    assert max_abs(xx.float(), ref) <= 2 ** -7 * ref.abs().max().item()


def test_pair_transition_residual_and_rowwise(gpu_device):
    m = _transition(gpu_device, 128, 512)
    x = torch.randn(2, 30, 30, 128).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        upd = m(x)
        # row-wise op: a sub-batch gives identical bits
        assert torch.equal(m(x[1:2]), upd[1:2])
        xx = x.clone()
        _ops.launch_transition_pair(xx, *m.prepared_params(), xx, residual=True)
    ref = x.float() + upd.float()
    assert max_abs(xx.float(), ref) <= 2 ** -7 * ref.abs().max().item()


@pytest.mark.parametrize(
    "dim,hidden,out_dim,use_norm",
    [(512, 1024, 128, False), (512, 1024, 384, False), (96, 192, 96, True), (160, 320, 64, True)],
)
def test_transition_out_dim_and_any_width(gpu_device, dim, hidden, out_dim, use_norm):
    """Transition(dim, hidden, out_dim, use_norm) at the denoiser's mixer shapes (diffusion.py:623-634:
    dim = a_s + atom_s, out_dim = atom_s or a_s, no LayerNorm) and widths outside the fused kernel's set."""
    torch.manual_seed(3)
    m = Transition(dim, hidden, out_dim=out_dim, use_norm=use_norm)
    if use_norm:
        with torch.no_grad():
            m.norm.weight.normal_(1.0, 0.1)
            m.norm.bias.normal_(0.0, 0.1)
    m = m.to(gpu_device)
    x = torch.randn(3, 37, dim, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        got = m(x).float().cpu()
    assert got.shape == (3, 37, out_dim)
    want = oracle.transition(x.cpu(), state(m), use_norm=use_norm)
    _check(got, want, f"transition {dim}->{out_dim} hidden={hidden} norm={use_norm}")
