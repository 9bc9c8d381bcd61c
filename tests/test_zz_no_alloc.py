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
