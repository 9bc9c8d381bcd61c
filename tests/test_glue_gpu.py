"""HIP pair glue (distogram head, pairwise conditioning) vs the fp32 CPU oracle; trunk-embedding files."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.embeddings import TrunkEmbeddings
from bioemu2_amd.glue import DistogramModule, PairwiseConditioning
from bioemu2_amd.transition import Transition
from bioemu2_amd.residual import join_stream
from bioemu2_amd.workloads import init_module
from tests._helpers import max_abs, randomize_params, rel_l2, state

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("bf16_autocast")]

ATOL = 2e-2
RTOL_L2 = 1e-2


def _check(got, want, tag):
    """The bf16 bound: max-abs 2e-2 and rel-L2 1e-2 against the fp32 oracle."""
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f}", flush=True)
    assert err <= ATOL and rl2 <= RTOL_L2, (tag, err, rl2)


@pytest.mark.parametrize("B,N,bins", [(1, 37, 64), (2, 100, 64), (1, 64, 5), (1, 33, 128), (1, 1, 16)])
def test_distogram_matches_oracle_and_is_symmetric(gpu_device, B, N, bins):
    """fp32 z (bf16-representable values) gives the fp32 accumulator as output, held to the bound; bf16 z gives
    that output rounded once to bf16, bit for bit; both exactly symmetric."""
    torch.manual_seed(0)
    mod = randomize_params(DistogramModule(128, bins), 3).to(gpu_device)
    z = torch.randn(B, N, N, 128, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(gpu_device)
    got32 = mod(z.float())
    assert got32.dtype == torch.float32 and got32.shape == (B, N, N, bins)
    assert torch.equal(got32, got32.transpose(1, 2))
    _check(got32.cpu(), oracle.distogram(z.cpu(), state(mod)), f"distogram B={B} N={N} bins={bins}")
    got = mod(z)
    assert got.dtype == torch.bfloat16 and torch.equal(got, got32.to(torch.bfloat16))


@pytest.mark.parametrize("num_transitions,shape", [(2, (1, 48, 48)), (0, (2, 9, 9)), (1, (1, 100, 100))])
def test_pairwise_conditioning_matches_oracle(gpu_device, num_transitions, shape):
    """Each stage against the oracle on its own input (the projection, then every transition with its residual
    add; the stream is bf16 + int8 tail, the transition's LayerNorm reads its bf16 part), and the whole module
    against the oracle composition, all at the bf16 bound.  The module on bf16 inputs carries the same stream
    (fp32 inputs under bf16 autocast get it joined to fp32) and rounds it to bf16 once at the end."""
    torch.manual_seed(0)
    # the reference tests' recipe: default init, zero parameters re-drawn N(0, 0.02)
    mod = init_module(PairwiseConditioning(128, 128, num_transitions=num_transitions), 5).to(gpu_device)
    P = state(mod)
    g = torch.Generator().manual_seed(2)
    z = torch.randn(*shape, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    rel = torch.randn(*shape, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = mod(z.float(), rel.float())
    assert got.dtype == torch.float32
    # stage 0: LN over the concatenation + projection
    x = torch.empty(*shape, 128, dtype=torch.bfloat16, device=gpu_device)
    x_tail = torch.empty(x.shape, dtype=torch.int8, device=gpu_device)
    _ops.launch_pair_cond_proj(z, rel, *mod.prepared_params(), x, out_tail=x_tail)
    _check(join_stream(x, x_tail).cpu(), oracle.pairwise_conditioning(z.cpu(), rel.cpu(), P, 0),
           "pair_cond projection")
    # stages 1..T: x = transition(x) + x, in place on the stream
    for k, t in enumerate(mod.transitions):
        full, hi = join_stream(x, x_tail).cpu(), x.cpu()
        _ops.launch_transition_pair(x, *t.prepared_params(), x, residual=True, tail=x_tail)
        sub = {n[len(f"transitions.{k}."):]: v for n, v in P.items() if n.startswith(f"transitions.{k}.")}
        _check(join_stream(x, x_tail).cpu(), full + oracle.transition(hi, sub), f"pair_cond transition {k}")
    assert torch.equal(got, join_stream(x, x_tail))   # the module runs exactly these stages
    want = oracle.pairwise_conditioning(z.cpu(), rel.cpu(), P, num_transitions)
    _check(got.cpu(), want, f"pairwise conditioning T={num_transitions} {shape} composite")
    assert torch.equal(mod(z, rel), got.to(torch.bfloat16))   # bf16 in: the same stream, rounded once


def test_transition_hidden_two_x(gpu_device):
    """The conditioning transitions' shape (dim 128, hidden 256) through the drop-in Transition."""
    torch.manual_seed(0)
    m = randomize_params(Transition(128, 256), 4).to(gpu_device).eval()
    x = torch.randn(1, 40, 40, 128).to(torch.bfloat16).to(gpu_device)
    with torch.no_grad():
        got = m(x).float().cpu()
    _check(got, oracle.transition(x.cpu(), state(m)), "transition 128 -> 256")


def test_trunk_embeddings_from_gpu_round_trip(gpu_device, tmp_path):
    torch.manual_seed(0)
    dg = randomize_params(DistogramModule(128, 64), 3).to(gpu_device)
    z = torch.randn(1, 20, 20, 128).to(torch.bfloat16).to(gpu_device)
    e = TrunkEmbeddings(
        s_inputs=torch.randn(1, 20, 32, device=gpu_device),
        single=torch.randn(1, 20, 384, device=gpu_device).to(torch.bfloat16),
        pair=z,
        relative_position_encoding=torch.randn(1, 20, 20, 128, device=gpu_device).to(torch.bfloat16),
        distogram=dg(z),
    )
    path = tmp_path / "emb" / "embeddings.pt"
    e.save(path)
    loaded = TrunkEmbeddings.load(path, device=gpu_device)
    for name in TrunkEmbeddings.__dataclass_fields__:
        a, b = getattr(loaded, name), getattr(e, name)
        assert a.device == b.device and a.dtype == b.dtype and torch.equal(a, b)
