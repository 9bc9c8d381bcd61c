"""The allocation-free transition entry point against the workspace one, through the C ABI.

``bioemu_transition_pair_fwd_noalloc`` runs the kernels of
``bioemu_transition_pair_fwd`` with its scratch in a static device array, so
the two must agree bit for bit.  Two calls in a row, the second with a smaller
input (the array keeps the first call's contents), and a residual call with a
tail.
"""

from __future__ import annotations

import pytest
import torch

from bioemu2_amd import _ops
from bioemu2_amd._lib import check, lib
from bioemu2_amd.transition import Transition
from bioemu2_amd.workloads import init_module

pytestmark = pytest.mark.gpu


def _noalloc(x, params, out, tail=None, residual=False):
    nw, nb, w1, w2, w3 = params
    D, hidden = x.shape[-1], w1.shape[0]
    P = x.numel() // D
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = lib().bioemu_transition_pair_fwd_noalloc(
        ptr(x), ptr(nw), ptr(nb), ptr(w1), ptr(w2), ptr(w3), ptr(out), ptr(tail), P, D, hidden,
        int(nw is not None), int(residual), torch.cuda.current_stream(x.device).cuda_stream)
    check(rc, "bioemu_transition_pair_fwd_noalloc")
    return out


@pytest.mark.parametrize("dim", [128, 64])
def test_noalloc_matches_workspace_entry_point(gpu_device, dim):
    mod = init_module(Transition(dim, 4 * dim), 3).to(gpu_device)
    params = mod.prepared_params()
    g = torch.Generator().manual_seed(0)
    for rows in (5000, 777):  # second call smaller
        x = torch.randn(rows, dim, generator=g).to(torch.bfloat16).to(gpu_device)
        want = _ops.launch_transition_pair(x, *params, torch.empty_like(x))
        got = _noalloc(x, params, torch.empty_like(x))
        torch.cuda.synchronize()
        print(f"noalloc transition dim={dim} rows={rows}: equal={torch.equal(got, want)}", flush=True)
        assert torch.equal(got, want)


def test_noalloc_residual_tail_and_hidden2x(gpu_device):
    g = torch.Generator().manual_seed(1)
    for dim, hidden, rows in ((128, 512, 3000), (128, 256, 1000)):
        mod = init_module(Transition(dim, hidden), 4).to(gpu_device)
        params = mod.prepared_params()
        x = torch.randn(rows, dim, generator=g).to(gpu_device)
        hi, tail = _ops.stream_split(x)
        hi2, tail2 = hi.clone(), tail.clone()
        _ops.launch_transition_pair(hi, *params, hi, residual=True, tail=tail)
        _noalloc(hi2, params, hi2, tail2, residual=True)
        torch.cuda.synchronize()
        print(f"noalloc transition residual+tail hidden={hidden} rows={rows}", flush=True)
        assert torch.equal(hi, hi2) and torch.equal(tail, tail2)


def test_noalloc_rejects_unsupported(gpu_device):
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=gpu_device)
    w = torch.zeros(384, 96, dtype=torch.bfloat16, device=gpu_device)
    rc = lib().bioemu_transition_pair_fwd_noalloc(
        x.data_ptr(), None, None, w.data_ptr(), w.data_ptr(), w.data_ptr(), x.data_ptr(), None, 4, 96, 384, 0, 0,
        torch.cuda.current_stream().cuda_stream)
    assert rc == -2
    assert b"dim" in lib().bioemu_last_error()


def _graph_case(device, seed=5, rows=4096, dim=128):
    mod = init_module(Transition(dim, 4 * dim), seed).to(device)
    params = mod.prepared_params()
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, dim, generator=g).to(torch.bfloat16).to(device)
    return params, x


def test_noalloc_captured_in_a_graph_matches_eager_replays(gpu_device):
    """The allocation-free call captured in a HIP graph (after one eager call, so the scratch address is known):
    every replay equals the workspace entry point's eager result bit for bit, with eager calls of both entry
    points on other weights and shapes (which overwrite the shared scratch) and synchronisations between replays.
    The captured call refolds its weights into the scratch on every replay."""
    params, x = _graph_case(gpu_device)
    other, x2 = _graph_case(gpu_device, seed=6, rows=1000)
    want = _ops.launch_transition_pair(x, *params, torch.empty_like(x))
    out = torch.empty_like(x)
    _noalloc(x, params, out)   # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc(x, params, out)
    for k in range(4):
        out.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        print(f"noalloc graph replay {k}: equal={torch.equal(out, want)}", flush=True)
        assert torch.equal(out, want)
        scratch_user = _noalloc(x2, other, torch.empty_like(x2))   # overwrites the shared scratch eagerly
        assert torch.equal(scratch_user, _ops.launch_transition_pair(x2, *other, torch.empty_like(x2)))
        torch.cuda.synchronize()


_FIRST_CALL_CAPTURED = r"""
import torch
from tests.test_zz_no_alloc import _graph_case, _noalloc
from bioemu2_amd import _ops
dev = torch.device("cuda:0")
params, x = _graph_case(dev)
out = torch.empty_like(x)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    _noalloc(x, params, out)   # the process's first noalloc call: the scratch lookup happens under capture
want = _ops.launch_transition_pair(x, *params, torch.empty_like(x))
for k in range(3):
    out.fill_(0)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), k
print("first-call capture ok", flush=True)
"""


def test_noalloc_first_call_under_capture(gpu_device):
    """In a fresh process whose first allocation-free call is made under graph capture (the per-device scratch
    address is looked up inside the capture), the graph's replays equal the workspace entry point's result."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED], cwd=root, env=env, capture_output=True,
                       text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "first-call capture ok" in r.stdout
