"""HIP triangle attention vs the fp32 CPU oracle; bit-exact mask and padding invariance."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.strategy import make
from bioemu2_amd.triangle_attention import REGISTRY, TriangleAttentionHip
from tests._helpers import max_abs, rel_l2, state

pytestmark = pytest.mark.gpu

C, H = 128, 4
ATOL = 2e-2  # north_star bf16 tolerance vs the fp32 oracle
RTOL_L2 = 1e-2


def _module(starting: bool, device, seed: int = 7) -> TriangleAttentionHip:
    torch.manual_seed(seed)
    m = make(REGISTRY, "hip", starting=starting, c_z=C, num_heads=H)
    return m.to(device).eval()


def _inputs(n: int, device, seed: int = 0, p_valid: float = 0.8):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, C, generator=g).to(torch.bfloat16)
    mask = torch.rand(1, n, n, generator=g) < p_valid
    return z.to(device), mask.to(device)


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("n", [16, 37, 100, 160])
def test_matches_oracle(gpu_device, starting, n):
    m = _module(starting, gpu_device)
    z, mask = _inputs(n, gpu_device)
    with torch.no_grad():
        got = m(z, mask).float().cpu()
    want = oracle.triangle_attention(z.float().cpu(), mask.cpu(), state(m), H, starting)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"triatt starting={starting} n={n}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("starting", [True, False])
def test_token_padding_config_shape(gpu_device, starting):
    """Config-4 style: trailing padded tokens, pair mask = outer AND, N=300."""
    n, n_pad = 300, 30
    m = _module(starting, gpu_device)
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, C, generator=g).to(torch.bfloat16)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, n - n_pad:] = False
    pm = oracle.pair_mask_from_token_mask(tok)
    with torch.no_grad():
        got = m(z.to(gpu_device), pm.to(gpu_device)).float().cpu()
    want = oracle.triangle_attention(z.float(), pm, state(m), H, starting, row_chunk=50)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"triatt n=300 padded starting={starting}: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("starting", [True, False])
def test_config4_shape_n768(gpu_device, starting):
    """Config 4: N=768, last 76 tokens padded, pair mask = outer AND (oracle row-chunked)."""
    n, n_pad = 768, 76
    m = _module(starting, gpu_device)
    g = torch.Generator().manual_seed(0)
    z = torch.randn(1, n, n, C, generator=g).to(torch.bfloat16)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, n - n_pad:] = False
    pm = oracle.pair_mask_from_token_mask(tok)
    with torch.no_grad():
        got = m(z.to(gpu_device), pm.to(gpu_device)).float().cpu()
    want = oracle.triangle_attention(z.float(), pm, state(m), H, starting, row_chunk=64)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"triatt n=768 padded starting={starting}: max_abs={err:.3e} rel_l2={rl2:.3e}", flush=True)
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("starting", [True, False])
def test_config5_shape_n2048(gpu_device, starting):
    """Config 5's pair shape: N=2048 with the last 102 tokens padded (32 key blocks, the last one partly masked),
    starting and ending node, against the row-chunked fp32 oracle."""
    n, n_pad = 2048, 102
    print(f"triatt n=2048 starting={starting}: GPU", flush=True)
    m = _module(starting, gpu_device)
    g = torch.Generator().manual_seed(5)
    z = torch.randn(1, n, n, C, generator=g).to(torch.bfloat16)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, n - n_pad:] = False
    pm = oracle.pair_mask_from_token_mask(tok)
    with torch.no_grad():
        got = m(z.to(gpu_device), pm.to(gpu_device)).float().cpu()
    want = oracle.triangle_attention(z.float(), pm, state(m), H, starting, row_chunk=32)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"triatt n=2048 padded starting={starting}: max_abs={err:.3e} rel_l2={rl2:.3e}", flush=True)
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("starting", [True, False])
def test_masked_key_blocks_match_oracle(gpu_device, starting):
    """Frame rows whose valid keys sit in scattered 64-key blocks: the first block fully masked, holes of
    whole blocks, a single valid key, and rows with no valid key at all.  The kernel skips key blocks
    without a valid key (they add exact zeros) and gives a row without any its uniform mean of v; both
    against the oracle on every element."""
    n = 320                                     # 5 key blocks of 64
    g = torch.Generator().manual_seed(11)
    fm = torch.zeros(1, n, n, dtype=torch.bool)   # frame mask: [row i][key k]
    blocks = {0: [1, 3], 1: [0, 4], 2: [0, 1, 2, 3, 4], 3: [2], 4: []}
    for i in range(n):
        for kb in blocks[i % 5]:
            fm[0, i, 64 * kb:64 * kb + 64] = torch.rand(64, generator=g) < 0.7
        if i % 5 == 3:
            fm[0, i] = False
            fm[0, i, 130] = True
    mask = fm if starting else fm.transpose(1, 2).contiguous()
    m = _module(starting, gpu_device)
    z = torch.randn(1, n, n, C, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        got = m(z.to(gpu_device), mask.to(gpu_device)).float().cpu()
    want = oracle.triangle_attention(z.float(), mask, state(m), H, starting, row_chunk=80)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"triatt masked key blocks starting={starting}: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("starting", [True, False])
def test_masking_bit_exact(gpu_device, starting):
    """Values under masked pairs never reach valid outputs... except through
    their own row/col: for the starting node a masked pair (i,k) is a masked key
    of row i but still a query of row i and a bias source; so only change the
    pairs that are masked *and* lie in fully padded token rows/cols."""
    n, n_pad = 70, 9
    m = _module(starting, gpu_device)
    z, _ = _inputs(n, gpu_device)
    tok = torch.ones(1, n, dtype=torch.bool, device=gpu_device)
    tok[:, n - n_pad:] = False
    pm = tok[:, :, None] & tok[:, None, :]
    changed = z.clone()
    changed[~pm] = 1000.0
    with torch.no_grad():
        a = m(z, pm)
        b = m(changed, pm)
    assert torch.equal(a[pm], b[pm])


@pytest.mark.parametrize("starting", [True, False])
def test_padding_bit_exact(gpu_device, starting):
    n, pad = 90, 45  # crosses the 32-key block and 128-query tile boundaries
    m = _module(starting, gpu_device)
    z, mask = _inputs(n, gpu_device)
    pz = torch.full((1, n + pad, n + pad, C), 1000.0, dtype=z.dtype, device=gpu_device)
    pz[:, :n, :n] = z
    pmask = torch.zeros(1, n + pad, n + pad, dtype=torch.bool, device=gpu_device)
    pmask[:, :n, :n] = mask
    with torch.no_grad():
        a = m(z, mask)
        b = m(pz, pmask)[:, :n, :n]
    assert torch.equal(a, b)


@pytest.mark.parametrize("scale", [2.0, 10.0])
@pytest.mark.parametrize("starting", [True, False])
def test_running_max_moves_key_order_invariant(gpu_device, starting, scale):
    """Logits that rise with the key index by far more than 16 log2 units make the kernel leave its unshifted
    softmax or move its running max: the ascending order meets its larger logits in later 64-key blocks, the
    reversed token order (the same problem, relabelled) in the first block.  At scale 2 head 0's first block in
    ascending order has maxima in [-64, 16] (unshifted start, then a shift), reversed above 16 (shifted start);
    at scale 10 the ascending first block lies below -64 (shifted start at a negative max).  Relabelling every
    token is an exact symmetry of triangle attention, so the two runs must agree to the north_star bf16 bar.
    (Against the fp32 oracle these logits are not a fair case: the ×log2e bias is stored in bf16, whose
    rounding at |logit| ≈ 20 is worth several percent of an attention weight, in any bf16 implementation.)"""
    n = 250
    m = _module(starting, gpu_device)
    with torch.no_grad():
        m.proj_b.weight.mul_(scale)
    w = m.proj_b.weight[0].detach().float().cpu()
    g = torch.Generator().manual_seed(11)
    u = w - w.mean()
    u = u / u.std()
    v = torch.randn(C, generator=g)
    v = v - v.mean()
    v = v - (v @ u) / (u @ u) * u
    v = v / v.std()
    theta = torch.pi * (1.0 - torch.arange(n) / (n - 1))          # key k: bias of head 0 ~ -cos(pi k/(n-1))
    zk = torch.cos(theta)[:, None] * u + torch.sin(theta)[:, None] * v
    z = (zk[None, None] + 0.1 * torch.randn(1, n, n, C, generator=g)).to(torch.bfloat16)   # z[., j, k] ~ zk[k]
    if not starting:
        z = z.transpose(1, 2).contiguous()   # the ending node's bias reads z[k, j]
    # The construction does what it claims: head 0's bias (log2 units) rises by > 16 after the first key block.
    lnz = torch.nn.functional.layer_norm(zk, (C,))
    b2 = (lnz @ w) * 1.4426950408889634
    assert b2[64:].max() - b2[:64].max() > 24.0
    assert b2.max() > 16.0 and (b2[:64].max() < -64.0) == (scale > 5.0)
    mask = torch.ones(1, n, n, dtype=torch.bool)
    mask[:, :, 5] = False
    mask[:, 7, :] = False
    z, mask = z.to(gpu_device), mask.to(gpu_device)
    with torch.no_grad():
        fwd = m(z, mask).float()
        rev = m(z.flip(1, 2).contiguous(), mask.flip(1, 2).contiguous()).flip(1, 2).float()
    assert torch.isfinite(fwd).all()
    err, rl2 = max_abs(fwd, rev), rel_l2(fwd, rev)
    print(f"triatt rising logits starting={starting} scale={scale}: ascending vs reversed max_abs={err:.3e} rel_l2={rl2:.3e} "
          f"|out|max={fwd.abs().max():.3f}")
    assert err <= ATOL and rl2 <= RTOL_L2


def test_batch_equals_separate(gpu_device):
    m = _module(False, gpu_device)
    z0, m0 = _inputs(40, gpu_device, seed=1)
    z1, m1 = _inputs(40, gpu_device, seed=2)
    with torch.no_grad():
        both = m(torch.cat([z0, z1]), torch.cat([m0, m1]))
        assert torch.equal(both[0:1], m(z0, m0))
        assert torch.equal(both[1:2], m(z1, m1))


def test_deterministic(gpu_device):
    m = _module(True, gpu_device)
    z, mask = _inputs(130, gpu_device)
    with torch.no_grad():
        assert torch.equal(m(z, mask), m(z, mask))


@pytest.mark.parametrize("starting", [True, False])
def test_fused_residual_in_place(gpu_device, starting):
    m = _module(starting, gpu_device)
    z, mask = _inputs(64, gpu_device)
    with torch.no_grad():
        upd = m(z, mask)
        zz = z.clone()
        _ops.launch_triatt(zz, _ops.mask_u8(mask), *m.prepared_params(), zz, starting, residual=True)
    ref = z.float() + upd.float()
    assert max_abs(zz.float(), ref) <= 2 ** -7 * ref.abs().max().item()


def test_rejects_unsupported_heads(gpu_device):
    m = TriangleAttentionHip(c_z=C, num_heads=8).to(gpu_device)
    with pytest.raises(ValueError):
        m(torch.zeros(1, 8, 8, C, device=gpu_device), torch.ones(1, 8, 8, dtype=torch.bool, device=gpu_device))
