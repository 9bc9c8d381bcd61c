"""Full Pairformer block on the GPU vs the fp32 CPU oracle composition.

The block carries its residual streams with int8 tails (~16 significant bits)
and returns fp32 for fp32 inputs, so it is held to the bf16 bound itself:
max-abs <= 2e-2 and rel-L2 <= 1e-2 on every valid element, at the headline
shape (N = 768, 76 padded tokens) too.  The tests run under bf16 autocast (the
reference trunk's policy), which fp32 inputs need.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd.pairformer import PairformerBlockHip
from bioemu2_amd.workloads import init_module
from tests._helpers import max_abs, rel_l2, state

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("bf16_autocast")]

MAX_ABS = 2e-2   # north_star bf16 bound
REL_L2 = 1e-2


def _block(device, seed=0):
    torch.manual_seed(seed)
    return init_module(PairformerBlockHip(), seed).to(device).eval()


def _inputs(n, n_pad, device, seed=0, dtype=torch.float32):
    """Seeded z, s ~ N(0, 1) (bf16-representable values, so the oracle sees the GPU's exact inputs)."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16).to(dtype)
    s = torch.randn(1, n, 384, generator=g).to(torch.bfloat16).to(dtype)
    tok = torch.ones(1, n, dtype=torch.bool)
    if n_pad:
        tok[:, n - n_pad:] = False
    return s.to(device), z.to(device), tok.to(device)


def _check(name, got, want, sel):
    g, w = got.float().cpu()[sel], want[sel]
    err, rl2 = max_abs(g, w), rel_l2(g, w)
    print(f"{name}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={w.abs().max():.2f}", flush=True)
    assert err <= MAX_ABS and rl2 <= REL_L2, (name, err, rl2)


@pytest.mark.parametrize("n,n_pad", [(64, 0), (100, 10), (768, 76)])
def test_block_matches_oracle(gpu_device, n, n_pad):
    blk = _block(gpu_device)
    s, z, tok = _inputs(n, n_pad, gpu_device)
    print(f"block n={n} pad={n_pad}: GPU", flush=True)
    s_got, z_got = blk(s, z, tok)
    assert s_got.dtype == torch.float32 and z_got.dtype == torch.float32
    print(f"block n={n} pad={n_pad}: oracle", flush=True)
    chunk = 64 if n > 256 else None
    s_want, z_want = oracle.pairformer_block(s.cpu(), z.cpu(), tok.cpu(), state(blk), triatt_row_chunk=chunk)
    pm = oracle.pair_mask_from_token_mask(tok.cpu())
    _check(f"block n={n} z", z_got, z_want, pm)
    _check(f"block n={n} s", s_got, s_want, tok.cpu())


def test_block_bf16_inputs_round_once(gpu_device):
    """bf16 in, bf16 out: the stream is carried with tails and rounded once, so the result is the fp32
    path's result rounded to bf16, bit for bit."""
    blk = _block(gpu_device)
    s, z, tok = _inputs(80, 8, gpu_device)
    s32, z32 = blk(s, z, tok)
    s16, z16 = blk(s.to(torch.bfloat16), z.to(torch.bfloat16), tok)
    assert s16.dtype == torch.bfloat16 and z16.dtype == torch.bfloat16
    assert torch.equal(s16, s32.to(torch.bfloat16)) and torch.equal(z16, z32.to(torch.bfloat16))


def test_block_padding_bit_exact(gpu_device):
    blk = _block(gpu_device)
    n, pad = 70, 30
    s, z, tok = _inputs(n, 0, gpu_device)
    ps = torch.cat([s, torch.full((1, pad, 384), 3.0, dtype=s.dtype, device=gpu_device)], 1)
    pz = torch.full((1, n + pad, n + pad, 128), 1000.0, dtype=z.dtype, device=gpu_device)
    pz[:, :n, :n] = z
    ptok = torch.cat([tok, torch.zeros(1, pad, dtype=torch.bool, device=gpu_device)], 1)
    sa, za = blk(s, z, tok)
    sb, zb = blk(ps, pz, ptok)
    assert torch.equal(za, zb[:, :n, :n])
    assert torch.equal(sa, sb[:, :n])


def test_block_inplace_matches_out_of_place(gpu_device):
    blk = _block(gpu_device)
    s, z, tok = _inputs(48, 4, gpu_device)
    s_new, z_new = blk(s, z, tok)
    from bioemu2_amd.residual import join_stream, split_stream

    (s2, st), (z2, zt) = split_stream(s), split_stream(z)
    blk.forward_(s2, z2, tok, st, zt)
    assert torch.equal(join_stream(s2, st), s_new) and torch.equal(join_stream(z2, zt), z_new)


def test_block_two_masks_same_shape(gpu_device):
    """Two calls with different masks of the same shape, the first mask freed before the second call
    (the allocator may hand the second mask the first one's address): each result equals a fresh
    block's result for its own mask."""
    blk = _block(gpu_device)
    s, z, _ = _inputs(64, 0, gpu_device)

    def mask(n_pad):
        m = torch.ones(1, 64, dtype=torch.bool)
        m[:, 64 - n_pad:] = False
        return m.to(gpu_device)

    m1 = mask(5)
    r1 = blk(s, z, m1)
    del m1
    torch.cuda.synchronize()
    r2 = blk(s, z, mask(17))
    f1 = _block(gpu_device)(s, z, mask(5))
    f2 = _block(gpu_device)(s, z, mask(17))
    assert torch.equal(r1[1], f1[1]) and torch.equal(r1[0], f1[0])
    assert torch.equal(r2[1], f2[1]) and torch.equal(r2[0], f2[0])
    assert not torch.equal(r1[1], r2[1])


def test_block_config5_size_padding_invariant(gpu_device):
    """Config 5 shape (N = 2048, 102 padded tokens): the valid region is bit-identical when every padded
    token's s and every pair touching a padded token in z change, and all outputs are finite."""
    blk = _block(gpu_device)
    n, pad = 2048, 102
    s, z, tok = _inputs(n, pad, gpu_device, seed=5, dtype=torch.bfloat16)
    s2, z2 = s.clone(), z.clone()
    s2[:, n - pad:] = 7.0
    z2[:, n - pad:] = -5.0
    z2[:, :, n - pad:] = 3.0
    with torch.no_grad():
        blk.forward_(s, z, tok)
        blk.forward_(s2, z2, tok)
    v = n - pad
    assert torch.isfinite(z[:, :v, :v].float()).all() and torch.isfinite(s[:, :v].float()).all()
    assert torch.equal(z[:, :v, :v], z2[:, :v, :v])
    assert torch.equal(s[:, :v], s2[:, :v])


def test_block_n3072_padding_invariant(gpu_device):
    """One block at N = 3072 (the reference's single-GPU capacity point, docs/context-parallel-sampling.md:
    115-117; 154 padded tokens): outputs finite, and the valid region bit-identical when every padded token's
    s and every pair touching a padded token change."""
    blk = _block(gpu_device)
    n, pad = 3072, 154
    s, z, tok = _inputs(n, pad, gpu_device, seed=9, dtype=torch.bfloat16)
    v = n - pad
    results = []
    for k in range(2):
        if k:
            s[:, v:] = 7.0
            z[:, v:] = -5.0
            z[:, :, v:] = 3.0
        s2, z2 = s.clone(), z.clone()
        print(f"block n={n} pass {k}", flush=True)
        with torch.no_grad():
            blk.forward_(s2, z2, tok)
        torch.cuda.synchronize()
        results.append((s2[:, :v].clone(), z2[:, :v, :v].clone()))
        del s2, z2
    (sa, za), (sb, zb) = results
    assert torch.isfinite(za.float()).all() and torch.isfinite(sa.float()).all()
    assert torch.equal(za, zb) and torch.equal(sa, sb)


def test_trunk_48_blocks_config5(gpu_device):
    """Config 5: all 48 blocks at N = 2048 (102 padded tokens), residual streams with tails, one shared
    workspace.  The whole trunk's valid outputs are finite and bit-identical when every padded token's s
    and every pair touching a padded token in z change."""
    from bioemu2_amd.residual import join_stream, split_stream

    n, pad, nblk = 2048, 102, 48
    blocks = [_block(gpu_device, seed=k) for k in range(nblk)]
    ws = torch.empty(blocks[0].workspace_bytes(1, n), dtype=torch.uint8, device=gpu_device)
    s, z, tok = _inputs(n, pad, gpu_device, seed=5, dtype=torch.bfloat16)
    s2, z2 = s.clone(), z.clone()
    s2[:, n - pad:] = 7.0
    z2[:, n - pad:] = -5.0
    z2[:, :, n - pad:] = 3.0
    results = []
    for s_in, z_in in ((s, z), (s2, z2)):
        (sh, st), (zh, zt) = split_stream(s_in), split_stream(z_in)
        del s_in, z_in
        for k, blk in enumerate(blocks):
            blk.forward_(sh, zh, tok, st, zt, ws=ws)
        torch.cuda.synchronize()
        print(f"trunk pass done ({nblk} blocks)", flush=True)
        v = n - pad
        results.append((join_stream(sh[:, :v], st[:, :v]),
                        join_stream(zh[:, :v, :v].contiguous(), zt[:, :v, :v].contiguous())))
        del sh, st, zh, zt
    (sa, za), (sb, zb) = results
    assert torch.isfinite(za).all() and torch.isfinite(sa).all()
    print(f"trunk |z|max={za.abs().max().item():.2f} |s|max={sa.abs().max().item():.2f}", flush=True)
    assert torch.equal(za, zb) and torch.equal(sa, sb)


def test_block_precision_follows_autocast(gpu_device):
    """fp32 inputs with autocast off take the fp32 path (no bf16 rounding of the streams: the result differs
    from the bf16 path's); bf16 inputs with autocast off select the bf16 path explicitly."""
    blk = _block(gpu_device)
    s, z, tok = _inputs(32, 0, gpu_device)
    s_mixed, z_mixed = blk(s, z, tok)                       # bf16 autocast (module fixture)
    with torch.autocast("cuda", enabled=False):
        s32, z32 = blk(s, z, tok)
        s16, z16 = blk(s.to(torch.bfloat16), z.to(torch.bfloat16), tok)
    assert s32.dtype == torch.float32 and z16.dtype == torch.bfloat16
    assert not torch.equal(z32, z_mixed)
    assert torch.equal(z16, z_mixed.to(torch.bfloat16)) and torch.equal(s16, s_mixed.to(torch.bfloat16))
