"""HIP pair glue (distogram head, pairwise conditioning) vs the fp32 CPU oracle; trunk-embedding files."""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.embeddings import TrunkEmbeddings
from bioemu2_amd.glue import DistogramModule, PairwiseConditioning
from bioemu2_amd.transition import Transition
from tests._helpers import max_abs, randomize_params, rel_l2, state

pytestmark = pytest.mark.gpu

ATOL = 2e-2
RTOL_L2 = 1e-2


def _check(got, want, tag, roundings=0):
    """max-abs 2e-2 and rel-L2 1e-2, plus 2^-9 |want| per bf16 rounding of a stored intermediate or
    output whose magnitude exceeds ~1 (the stored bf16 value itself carries that error)."""
    err, rl2 = max_abs(got, want), rel_l2(got, want)
    excess = ((got - want).abs() - (ATOL + roundings * 2.0 ** -9 * want.abs())).max().item()
    print(f"{tag}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={want.abs().max():.3f} excess={excess:.3e}")
    assert excess <= 0.0 and rl2 <= RTOL_L2


@pytest.mark.parametrize("B,N,bins", [(1, 37, 64), (2, 100, 64), (1, 64, 5), (1, 33, 128), (1, 1, 16)])
def test_distogram_matches_oracle_and_is_symmetric(gpu_device, B, N, bins):
    torch.manual_seed(0)
    mod = randomize_params(DistogramModule(128, bins), 3).to(gpu_device)
    z = torch.randn(B, N, N, 128, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(gpu_device)
    got = mod(z)
    assert got.dtype == torch.bfloat16 and got.shape == (B, N, N, bins)
    assert torch.equal(got, got.transpose(1, 2))
    want = oracle.distogram(z.cpu(), state(mod))
    # stored bf16: z + z^T (the reference's bf16 add) and the output
    _check(got.float().cpu(), want, f"distogram B={B} N={N} bins={bins}", roundings=2)


@pytest.mark.parametrize("num_transitions,shape", [(2, (1, 48, 48)), (0, (2, 9, 9)), (1, (1, 100, 100))])
def test_pairwise_conditioning_matches_oracle(gpu_device, num_transitions, shape):
    """Each stage against the oracle on the same bf16 input (the projection, then every transition with its
    residual add), and the whole module against the oracle composition by rel-L2: stacking residual
    transitions grows the bf16 error of the composite with the number of stages."""
    torch.manual_seed(0)
    mod = randomize_params(PairwiseConditioning(128, 128, num_transitions=num_transitions), 5).to(gpu_device)
    P = state(mod)
    g = torch.Generator().manual_seed(2)
    z = torch.randn(*shape, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    rel = torch.randn(*shape, 128, generator=g).to(torch.bfloat16).to(gpu_device)
    got = mod(z, rel)
    # stage 0: LN over the concatenation + projection
    x = torch.empty(*shape, 128, dtype=torch.bfloat16, device=gpu_device)
    _ops.launch_pair_cond_proj(z, rel, *mod.prepared_params(), x)
    _check(x.float().cpu(), oracle.pairwise_conditioning(z.cpu(), rel.cpu(), P, 0), "pair_cond projection", 1)
    # stages 1..T: x = transition(x) + x
    for k, t in enumerate(mod.transitions):
        y = x.clone()
        _ops.launch_transition_pair(y, *t.prepared_params(), y, residual=True)
        sub = {n[len(f"transitions.{k}."):]: v for n, v in P.items() if n.startswith(f"transitions.{k}.")}
        want = x.float().cpu() + oracle.transition(x.cpu(), sub)
        _check(y.float().cpu(), want, f"pair_cond transition {k}", 1)
        x = y
    assert torch.equal(got, x)   # the module runs exactly these stages
    want = oracle.pairwise_conditioning(z.cpu(), rel.cpu(), P, num_transitions)
    rl2 = rel_l2(got.float().cpu(), want)
    print(f"pairwise conditioning T={num_transitions} {shape}: composite rel_l2={rl2:.3e} "
          f"max_abs={max_abs(got.float().cpu(), want):.3e}")
    assert rl2 <= RTOL_L2


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
