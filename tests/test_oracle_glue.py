"""Pins oracle.distogram and oracle.pairwise_conditioning (CPU), and the trunk-embedding file format.

distogram follows biomoa/modules/embedders.py:191-206; pairwise_conditioning
follows biomoa/modules/diffusion.py:509-535; TrunkEmbeddings follows
biomoa/models/score_model.py:50-78 and its tests (tests/test_sampling.py:936-959).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from bioemu2_amd.embeddings import TrunkEmbeddings
from bioemu2_amd.glue import DistogramModule, PairwiseConditioning
from tests._helpers import np_ln, np_params, np_sigmoid, randomize_params, state


def _silu(x):
    return x * np_sigmoid(x)


def test_distogram_matches_brute_force():
    torch.manual_seed(0)
    P = state(randomize_params(DistogramModule(8, 5), 1))
    z = torch.randn(2, 6, 6, 8, generator=torch.Generator().manual_seed(2))
    got = oracle.distogram(z, P).numpy()
    Pn = np_params(P)
    zn = z.double().numpy()
    want = np.zeros((2, 6, 6, 5))
    for b in range(2):
        for i in range(6):
            for j in range(6):
                want[b, i, j] = (zn[b, i, j] + zn[b, j, i]) @ Pn["distogram.weight"].T + Pn["distogram.bias"]
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


def test_distogram_is_exactly_symmetric_and_transpose_matters():
    P = state(randomize_params(DistogramModule(8, 5), 1))
    z = torch.randn(1, 7, 7, 8, generator=torch.Generator().manual_seed(3))
    out = oracle.distogram(z, P)
    assert torch.equal(out, out.transpose(1, 2))
    planted = z @ P["distogram.weight"].T + P["distogram.bias"]   # the head without z^T
    assert not torch.allclose(planted, planted.transpose(1, 2), atol=1e-3)


def _pc_brute(z, rel, P, num_transitions):
    P = np_params(P)
    x = np.concatenate([z.double().numpy(), rel.double().numpy()], axis=-1)
    out = np.zeros(x.shape[:-1] + (P["dim_pairwise_init_proj.1.weight"].shape[0],))
    for idx in np.ndindex(*x.shape[:-1]):
        v = np_ln(x[idx], P["dim_pairwise_init_proj.0.weight"], P["dim_pairwise_init_proj.0.bias"])
        v = P["dim_pairwise_init_proj.1.weight"] @ v
        for k in range(num_transitions):
            p = f"transitions.{k}."
            t = np_ln(v, P[p + "norm.weight"], P[p + "norm.bias"])
            v = P[p + "fc3.weight"] @ (_silu(P[p + "fc1.weight"] @ t) * (P[p + "fc2.weight"] @ t)) + v
        out[idx] = v
    return out


@pytest.mark.parametrize("num_transitions", [0, 2])
def test_pairwise_conditioning_matches_brute_force(num_transitions):
    torch.manual_seed(0)
    m = randomize_params(PairwiseConditioning(8, 6, a_z=10, num_transitions=num_transitions), 4)
    P = state(m)
    g = torch.Generator().manual_seed(5)
    z = torch.randn(1, 4, 4, 8, generator=g)
    rel = torch.randn(1, 4, 4, 6, generator=g)
    got = oracle.pairwise_conditioning(z, rel, P, num_transitions).numpy()
    np.testing.assert_allclose(got, _pc_brute(z, rel, P, num_transitions), atol=2e-5, rtol=1e-5)


def test_pairwise_conditioning_concatenation_order():
    """z_trunk fills the first token_z channels: swapping the inputs changes the result."""
    m = randomize_params(PairwiseConditioning(8, 8, num_transitions=1), 6)
    P = state(m)
    g = torch.Generator().manual_seed(7)
    z = torch.randn(1, 3, 3, 8, generator=g)
    rel = torch.randn(1, 3, 3, 8, generator=g)
    a = oracle.pairwise_conditioning(z, rel, P, 1)
    b = oracle.pairwise_conditioning(rel, z, P, 1)
    assert not torch.allclose(a, b, atol=1e-3)


def _embeddings(dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(0)
    return TrunkEmbeddings(
        s_inputs=torch.randn(1, 5, 12, generator=g).to(dtype),
        single=torch.randn(1, 5, 8, generator=g).to(dtype),
        pair=torch.randn(1, 5, 5, 4, generator=g).to(dtype),
        relative_position_encoding=torch.randn(1, 5, 5, 4, generator=g).to(dtype),
        distogram=torch.randn(1, 5, 5, 3, generator=g).to(dtype),
    )


def test_trunk_embeddings_round_trip_and_format(tmp_path):
    e = _embeddings()
    path = tmp_path / "saved" / "embeddings.pt"
    e.save(path)
    assert path.is_file()
    loaded = TrunkEmbeddings.load(path, device=torch.device("cpu"))
    for name in TrunkEmbeddings.__dataclass_fields__:
        assert torch.equal(getattr(loaded, name), getattr(e, name))
        assert getattr(loaded, name).dtype == torch.bfloat16
    # the file is a plain dict of exactly the five host tensors (what the reference's load accepts)
    raw = torch.load(path, map_location="cpu", weights_only=True)
    assert isinstance(raw, dict)
    assert set(raw) == {"s_inputs", "single", "pair", "relative_position_encoding", "distogram"}
    assert all(isinstance(v, torch.Tensor) and v.device.type == "cpu" for v in raw.values())


def test_trunk_embeddings_refuses_to_overwrite(tmp_path):
    path = tmp_path / "embeddings.pt"
    path.write_bytes(b"keep me")
    with pytest.raises(FileExistsError, match="existing file"):
        _embeddings().save(path)
    assert path.read_bytes() == b"keep me"


def test_trunk_embeddings_rejects_invalid_files(tmp_path):
    bad_keys = tmp_path / "a.pt"
    torch.save({"single": torch.zeros(1)}, bad_keys)
    with pytest.raises(ValueError, match="Invalid trunk embeddings"):
        TrunkEmbeddings.load(bad_keys, device=torch.device("cpu"))
    not_dict = tmp_path / "b.pt"
    torch.save([torch.zeros(1)], not_dict)
    with pytest.raises(ValueError, match="Invalid trunk embeddings"):
        TrunkEmbeddings.load(not_dict, device=torch.device("cpu"))
    non_tensor = tmp_path / "c.pt"
    d = {k: torch.zeros(1) for k in TrunkEmbeddings.__dataclass_fields__}
    d["pair"] = 3
    torch.save(d, non_tensor)
    with pytest.raises(ValueError, match="Invalid trunk embeddings"):
        TrunkEmbeddings.load(non_tensor, device=torch.device("cpu"))
