"""HIP TriMul vs the fp32 CPU oracle, plus bit-exact mask/padding invariance on the GPU."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.strategy import make
from bioemu2_amd.triangle_multiplication import REGISTRY, TriangleMultiplicationHip
from tests._helpers import max_abs, redraw_zero_params, rel_l2, state

pytestmark = pytest.mark.gpu

D = 128
# north_star tolerance for bf16 vs the fp32 reference
ATOL = 2e-2
RTOL_L2 = 1e-2


def _module(mode: str, device) -> TriangleMultiplicationHip:
    torch.manual_seed(42)
    m = make(REGISTRY, "cueq", dim=D, mode=mode, tile_size=None, matmul_precision="ieee")
    return redraw_zero_params(m).to(device).eval()


def _inputs(n: int, device, seed: int = 0, p_valid: float = 0.75):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, n, n, D, generator=g).to(torch.bfloat16)
    mask = torch.rand(1, n, n, generator=g) < p_valid
    return x.to(device), mask.to(device)


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
@pytest.mark.parametrize("n", [16, 37, 130, 256])
def test_matches_oracle(gpu_device, mode, n):
    m = _module(mode, gpu_device)
    x, mask = _inputs(n, gpu_device)
    with torch.no_grad():
        got = m(x, mask).float().cpu()
    want = oracle.trimul(x.float().cpu(), mask.cpu(), state(m), mode)
    assert want.abs().max() > 0
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"trimul {mode} n={n}: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_matches_oracle_n768_token_padding(gpu_device, mode):
    """Config 4 shape: N=768, last 76 tokens padded, pair mask = outer AND."""
    n = 768
    m = _module(mode, gpu_device)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, n, n, D, generator=g).to(torch.bfloat16)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, n - 76:] = False
    pm = oracle.pair_mask_from_token_mask(tok)
    with torch.no_grad():
        got = m(x.to(gpu_device), pm.to(gpu_device)).float().cpu()
    want = oracle.trimul(x.float(), pm, state(m), mode)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"trimul {mode} n=768: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_matches_oracle_n2048_token_padding(gpu_device, mode):
    """Config 5's pair shape: N=2048, last 102 tokens padded (planes padded to 2048, eight 256-wide contraction
    tiles), both directions, against the fp32 oracle."""
    n = 2048
    print(f"trimul {mode} n=2048: GPU", flush=True)
    m = _module(mode, gpu_device)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, n, n, D, generator=g).to(torch.bfloat16)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, n - 102:] = False
    pm = oracle.pair_mask_from_token_mask(tok)
    with torch.no_grad():
        got = m(x.to(gpu_device), pm.to(gpu_device)).float().cpu()
    want = oracle.trimul(x.float(), pm, state(m), mode)
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"trimul {mode} n=2048: max_abs={err:.3e} rel_l2={rl2:.3e}", flush=True)
    assert err <= ATOL and rl2 <= RTOL_L2


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_masking_bit_exact(gpu_device, mode):
    m = _module(mode, gpu_device)
    x, mask = _inputs(70, gpu_device)
    changed = x.clone()
    changed[~mask] = 1000.0
    with torch.no_grad():
        a = m(x, mask)
        b = m(changed, mask)
    assert torch.equal(a[mask], b[mask])


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_padding_bit_exact(gpu_device, mode):
    n, pad = 200, 100  # the contraction pads N to a multiple of 256: 200 -> 256, 300 -> 512
    m = _module(mode, gpu_device)
    x, mask = _inputs(n, gpu_device)
    px = torch.full((1, n + pad, n + pad, D), 1000.0, dtype=x.dtype, device=gpu_device)
    px[:, :n, :n] = x
    pmask = torch.zeros(1, n + pad, n + pad, dtype=torch.bool, device=gpu_device)
    pmask[:, :n, :n] = mask
    with torch.no_grad():
        a = m(x, mask)
        b = m(px, pmask)[:, :n, :n]
    assert torch.equal(a, b)


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_projection_workgroup_sizes_bit_exact(gpu_device, mode):
    """The input projection's workgroup size is chosen from the tile count: N = 512 runs 8-wave workgroups,
    the same problem with 88 masked tokens appended (N = 600, padded to 768) runs 12-wave ones.  A tile's result
    does not depend on which wave computes it and padded k columns are zeros, so the valid region must agree
    bit for bit."""
    n, pad = 512, 88
    m = _module(mode, gpu_device)
    x, mask = _inputs(n, gpu_device, seed=6)
    px = torch.full((1, n + pad, n + pad, D), 7.0, dtype=x.dtype, device=gpu_device)
    px[:, :n, :n] = x
    pmask = torch.zeros(1, n + pad, n + pad, dtype=torch.bool, device=gpu_device)
    pmask[:, :n, :n] = mask
    with torch.no_grad():
        a = m(x, mask)
        b = m(px, pmask)[:, :n, :n]
    assert torch.equal(a, b)


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_n3072_matches_unpadded_n2816(gpu_device, mode):
    """N = 3072, the reference's single-GPU capacity point (docs/context-parallel-sampling.md:115-117): the
    contraction planes (128 x 3072^2 bf16, 2.4 GB per operand) pass 2^31 bytes, so tile offsets into them need
    the full 32-bit range.  With the last 256 tokens masked, the valid region must equal, bit for bit, the same
    problem at N = 2816 (planes below 2^31 bytes); all outputs finite."""
    n, pad = 2816, 256
    m = _module(mode, gpu_device)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, n + pad, n + pad, D, generator=g).to(torch.bfloat16).to(gpu_device)
    tok = torch.ones(1, n + pad, dtype=torch.bool, device=gpu_device)
    tok[:, n:] = False
    pmask = tok[:, :, None] & tok[:, None, :]
    print(f"trimul {mode} N={n + pad}", flush=True)
    with torch.no_grad():
        b = m(x, pmask)
        assert torch.isfinite(b).all()
        b = b[:, :n, :n].clone()
        xs = x[:, :n, :n].contiguous()
        del x, pmask
        torch.cuda.empty_cache()
        print(f"trimul {mode} N={n}", flush=True)
        a = m(xs, torch.ones(1, n, n, dtype=torch.bool, device=gpu_device))
    assert torch.equal(a, b)


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_n4352_matches_unpadded_n4096(gpu_device, mode):
    """Past N = 4096 (the reference runs its tiled kernel beyond 5000 tokens, triangle_multiplication.py:355-367):
    the 128 contraction planes of an N = 4352 problem span 4.8 GB, more than a 32-bit offset reaches from one base.
    With the last 256 tokens masked, the valid region must equal, bit for bit, the same problem at N = 4096; all
    outputs finite."""
    n, pad = 4096, 256
    m = _module(mode, gpu_device)
    g = torch.Generator(device=gpu_device).manual_seed(11)
    x = torch.randn(1, n + pad, n + pad, D, generator=g, device=gpu_device, dtype=torch.bfloat16)
    tok = torch.ones(1, n + pad, dtype=torch.bool, device=gpu_device)
    tok[:, n:] = False
    pmask = tok[:, :, None] & tok[:, None, :]
    print(f"trimul {mode} N={n + pad}", flush=True)
    with torch.no_grad():
        b = m(x, pmask)
        assert torch.isfinite(b).all()
        b = b[:, :n, :n].clone()
        xs = x[:, :n, :n].contiguous()
        del x, pmask
        torch.cuda.empty_cache()
        print(f"trimul {mode} N={n}", flush=True)
        a = m(xs, torch.ones(1, n, n, dtype=torch.bool, device=gpu_device))
    assert torch.equal(a, b)


def test_rejects_n_past_the_offset_range(gpu_device):
    """N = 9728 would need offsets past 32 bits in the output stage: the C entry point refuses the shape before it
    reads any argument buffer or launches anything (the buffers passed here are small on purpose)."""
    from bioemu2_amd._lib import lib

    buf = torch.zeros(1 << 16, dtype=torch.bfloat16, device=gpu_device)
    p = buf.data_ptr()
    rc = lib().bioemu_trimul_fwd(p, p, p, p, p, p, p, p, p, p, p, None, p, buf.numel() * 2, 1, 9728, D, 1, 0,
                                 torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"N <= 9472" in lib().bioemu_last_error()


def test_batch_equals_separate(gpu_device):
    m = _module("incoming", gpu_device)
    x0, m0 = _inputs(48, gpu_device, seed=1)
    x1, m1 = _inputs(48, gpu_device, seed=2)
    with torch.no_grad():
        both = m(torch.cat([x0, x1]), torch.cat([m0, m1]))
        assert torch.equal(both[0:1], m(x0, m0))
        assert torch.equal(both[1:2], m(x1, m1))


def test_deterministic(gpu_device):
    m = _module("outgoing", gpu_device)
    x, mask = _inputs(130, gpu_device)
    with torch.no_grad():
        assert torch.equal(m(x, mask), m(x, mask))


@pytest.mark.parametrize("mode", ["outgoing", "incoming"])
def test_fused_residual_in_place(gpu_device, mode):
    m = _module(mode, gpu_device)
    x, mask = _inputs(64, gpu_device)
    with torch.no_grad():
        upd = m(x, mask)
        z = x.clone()
        _ops.launch_trimul(z, _ops.mask_u8(mask), *m.prepared_params(), z, mode == "outgoing", residual=True)
    ref = (x.float() + upd.float())
    assert max_abs(z.float(), ref) <= 2 ** -7 * ref.abs().max().item()


def test_rejects_cpu_tensors():
    m = TriangleMultiplicationHip(dim=D)
    with pytest.raises(RuntimeError):
        m(torch.zeros(1, 4, 4, D), torch.ones(1, 4, 4, dtype=torch.bool))


def test_rejects_unsupported_dim(gpu_device):
    """The bf16 path supports dim 128 only (the fp32 path takes any multiple of 32)."""
    m = TriangleMultiplicationHip(dim=64).to(gpu_device)
    with pytest.raises(ValueError):
        m(torch.zeros(1, 8, 8, 64, device=gpu_device, dtype=torch.bfloat16),
          torch.ones(1, 8, 8, dtype=torch.bool, device=gpu_device))


def test_fp32_autocast_selects_the_bf16_path(gpu_device):
    """fp32 inputs under bf16 autocast (the reference trunk's policy) take the bf16 path and return fp32: the bf16
    result of the same (bf16-representable) input, cast.  With autocast off they take the fp32 path
    (tests/test_fp32_gpu.py)."""
    m = _module("outgoing", gpu_device)
    x, mask = _inputs(40, gpu_device)
    with torch.no_grad():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got = m(x.float(), mask)
        want = m(x, mask)
    assert got.dtype == torch.float32 and torch.equal(got.to(torch.bfloat16), want)
