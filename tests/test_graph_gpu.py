"""The in-place Pairformer block captured in a HIP graph and replayed.

``PairformerBlockHip.forward_`` launches only kernels on torch's current
stream (no memsets, host copies or synchronisations) and reuses the workspace,
masks and prepared weights it cached on its first call, so after one eager
call at a shape it can be captured with ``torch.cuda.graph``.  Every replay
must be bit-identical to the eager block on the same inputs, with unrelated
eager work and synchronisations between replays.
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
    want = _eager(blk, s0, z0, tok, steps=2)  # also caches workspace, masks and weights

    s_g, z_g = s0.clone(), z0.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        blk.forward_(s_g, z_g, tok)
    torch.cuda.synchronize()

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
        torch.cuda.synchronize()

    # Chained replays: the second replay reads the first one's in-place output.
    s_g.copy_(s0)
    z_g.copy_(z0)
    graph.replay()
    graph.replay()
    torch.cuda.synchronize()
    print("graph replay: two chained steps", flush=True)
    assert torch.equal(s_g, want[1][0]) and torch.equal(z_g, want[1][1])
