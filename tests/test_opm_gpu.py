"""HIP fused OuterProductMean vs the fp32 CPU oracle; exact masking and row-padding invariance."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.outer_product_mean import REGISTRY, OuterProductMeanHip
from bioemu2_amd.strategy import make
from tests._helpers import max_abs, rel_l2, state

pytestmark = pytest.mark.gpu

ATOL = 2e-2  # north_star bf16 bound (the reference's own bf16 OPM bound is 2.5e-2, test_outer_product_mean.py:22)
RTOL_L2 = 1e-2


def _module(device, seed=2) -> OuterProductMeanHip:
    torch.manual_seed(seed)
    m = make(REGISTRY, "vanilla", c_in=64, c_hidden=32, c_out=128)
    with torch.no_grad():
        m.proj_o.bias.normal_(0, 0.1)
    return m.to(device).eval()


def _inputs(B, S, N, device, p_row_masked=0.2, seed=0):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(B, S, N, 64, generator=g).to(torch.bfloat16)
    rows = torch.rand(B, S, generator=g) >= p_row_masked
    mask = rows[:, :, None].expand(B, S, N).clone()
    return m.to(device), mask.to(device)


def _check(got, want, tag):
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("B,S,N", [(1, 40, 16), (2, 300, 37), (1, 129, 64)])
def test_matches_oracle(gpu_device, B, S, N):
    m_ = _module(gpu_device)
    m, mask = _inputs(B, S, N, gpu_device)
    mask[:, 1, -3:] = False  # ragged entries inside a valid row (test_outer_product_mean.py:102-114)
    with torch.no_grad():
        got = m_(m, mask).float().cpu()
    want = oracle.outer_product_mean(m.cpu(), mask.cpu(), state(m_))
    _check(got, want, f"opm B={B} S={S} N={N}")


def test_config3_shape(gpu_device):
    """Config 3 shapes (S=1024, N=512, 20% rows masked): every output pair against the oracle."""
    m_ = _module(gpu_device)
    m, mask = _inputs(1, 1024, 512, gpu_device)
    with torch.no_grad():
        got = m_(m, mask).float().cpu()
    want = oracle.outer_product_mean(m.cpu(), mask.cpu(), state(m_), i_chunk=64)
    _check(got, want, "opm config3")


def test_2d_mask(gpu_device):
    """A [B,N] mask divides by 1 (outer_product_mean.py:69-70): the result is the sum over S, so S is kept
    small enough (6 rows) that outputs stay O(1) and the absolute bound is meaningful."""
    m_ = _module(gpu_device)
    m, _ = _inputs(1, 6, 20, gpu_device)
    tok = torch.ones(1, 20, dtype=torch.bool, device=gpu_device)
    tok[:, 15:] = False
    with torch.no_grad():
        got = m_(m, tok).float().cpu()
    want = oracle.outer_product_mean(m.cpu(), tok.cpu(), state(m_))
    _check(got, want, "opm 2d mask")


def test_all_rows_masked_gives_bias(gpu_device):
    m_ = _module(gpu_device)
    m, mask = _inputs(2, 30, 10, gpu_device)
    mask[1] = False
    with torch.no_grad():
        got = m_(m, mask)
    want_bias = m_.proj_o.bias.to(torch.bfloat16).expand(10, 10, 128)
    assert torch.equal(got[1], want_bias)


def test_masked_values_bit_exact(gpu_device):
    m_ = _module(gpu_device)
    m, mask = _inputs(1, 80, 24, gpu_device)
    mask[0, 3, 5:9] = False
    m2 = m.clone()
    m2[~mask] = 1000.0
    with torch.no_grad():
        assert torch.equal(m_(m, mask), m_(m2, mask))


def test_appended_masked_rows_bit_exact(gpu_device):
    """Row compaction makes masked MSA rows cost nothing and change no bit."""
    m_ = _module(gpu_device)
    m, mask = _inputs(1, 70, 30, gpu_device)
    pm = torch.cat([m, torch.randn(1, 40, 30, 64, device=gpu_device).to(m.dtype)], 1)
    pmask = torch.cat([mask, torch.zeros(1, 40, 30, dtype=torch.bool, device=gpu_device)], 1)
    with torch.no_grad():
        assert torch.equal(m_(m, mask), m_(pm, pmask))


def test_token_padding_bit_exact(gpu_device):
    m_ = _module(gpu_device)
    m, mask = _inputs(1, 60, 21, gpu_device)
    pm = torch.cat([m, torch.full((1, 60, 11, 64), 5.0, dtype=m.dtype, device=gpu_device)], 2)
    pmask = torch.cat([mask, torch.zeros(1, 60, 11, dtype=torch.bool, device=gpu_device)], 2)
    with torch.no_grad():
        assert torch.equal(m_(m, mask), m_(pm, pmask)[:, :21, :21])


def test_fused_residual_into_z(gpu_device):
    m_ = _module(gpu_device)
    m, mask = _inputs(1, 64, 32, gpu_device)
    z = torch.randn(1, 32, 32, 128, device=gpu_device).to(torch.bfloat16)
    with torch.no_grad():
        upd = m_(m, mask)
        zz = z.clone()
        mask3, mean_rows = _ops.opm_mask3(mask, 1, 64, 32)
        _ops.launch_opm(m, mask3, mean_rows, *m_.prepared_params(), out=zz, z_res=zz)
    ref = z.float() + upd.float()
    assert max_abs(zz.float(), ref) <= 2 ** -7 * ref.abs().max().item()
