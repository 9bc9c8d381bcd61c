"""The in-place Pairformer block captured in a HIP graph and replayed.

``PairformerBlockHip.forward_`` launches only kernels on torch's current
stream (no memsets, host copies or synchronisations).  ``capture()`` prepares
the weights outside the capture, gives the graph a workspace of its own and
keeps every buffer a replay touches alive.  Every replay must be bit-identical
to the eager block on the same inputs, with unrelated eager work, eager blocks
at a larger shape (which replace the block's cached workspace) and
synchronisations between replays; with and without residual tails.
"""

from __future__ import annotations

import pytest
import torch

from bioemu2_amd.pairformer import PairformerBlockHip
from bioemu2_amd.workloads import init_module

pytestmark = pytest.mark.gpu


def _setup(device, n=96, n_pad=6, seed=3):
    blk = init_module(PairformerBlockHip(), seed).to(device).eval()
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16).to(device)
    s = torch.randn(1, n, 384, generator=g).to(torch.bfloat16).to(device)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, n - n_pad:] = False
    return blk, s, z, tok.to(device)


def _eager(blk, s, z, tok, steps):
    s, z = s.clone(), z.clone()
    out = []
    for _ in range(steps):
        blk.forward_(s, z, tok)
        out.append((s.clone(), z.clone()))
    return out


def test_block_graph_replays_match_eager(gpu_device):
    blk, s0, z0, tok = _setup(gpu_device)
    want = _eager(blk, s0, z0, tok, steps=2)

    s_g, z_g = s0.clone(), z0.clone()
    graph = blk.capture(s_g, z_g, tok)
    torch.cuda.synchronize()
    big = _setup(gpu_device, n=160, n_pad=0)

    other = torch.randn(1 << 20, device=gpu_device)
    for rep in range(3):
        s_g.copy_(s0)
        z_g.copy_(z0)
        graph.replay()
        torch.cuda.synchronize()
        print(f"graph replay {rep}: fresh inputs", flush=True)
        assert torch.equal(s_g, want[0][0]) and torch.equal(z_g, want[0][1])
        # Eager work between replays: unrelated torch ops and an eager block on other buffers.
        other.mul_(1.0001).add_(0.5)
        _eager(blk, s0, z0, tok, steps=1)
        _eager(blk, big[1], big[2], big[3], steps=1)
        torch.cuda.synchronize()

    # Chained replays: the second replay reads the first one's in-place output.
    s_g.copy_(s0)
    z_g.copy_(z0)
    graph.replay()
    graph.replay()
    torch.cuda.synchronize()
    print("graph replay: two chained steps", flush=True)
    assert torch.equal(s_g, want[1][0]) and torch.equal(z_g, want[1][1])


def test_block_graph_with_tails(gpu_device):
    """The tail-carrying stream under a graph: replays equal the eager ``forward_`` with tails, bit for bit."""
    from bioemu2_amd.residual import split_stream

    blk, s0, z0, tok = _setup(gpu_device, n=64, n_pad=3, seed=4)
    s0, z0 = s0.float() * 1.37, z0.float() * 0.71           # values with non-zero tails
    (sh, st), (zh, zt) = split_stream(s0), split_stream(z0)
    e = [t.clone() for t in (sh, zh, st, zt)]
    blk.forward_(e[0], e[1], tok, e[2], e[3])
    g = [t.clone() for t in (sh, zh, st, zt)]
    graph = blk.capture(g[0], g[1], tok, g[2], g[3])
    for rep in range(2):
        for dst, src in zip(g, (sh, zh, st, zt)):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        print(f"graph replay {rep} with tails", flush=True)
        assert all(torch.equal(a, b) for a, b in zip(g, e))
