"""Pins the oracle's compositions (CPU): residual order and parameter routing.

``oracle.pairformer_block`` (AF3 suppl. Alg. 17), ``oracle.pairmixer_layer``
(pairmixer.py:446-456) and ``oracle.pairmixer_msa_layer`` (pairmixer.py:737-755)
are compositions of the per-op oracle functions, each pinned on its own
(tests/test_oracle_*.py).  What is left to pin is the composition itself:

* with every output projection zeroed, each op's update is exactly 0, so the
  composition must return its inputs bit for bit;
* with one output projection left non-zero, it must return input + that op's
  update, computed here from the op function and a sub-dict this test builds
  itself from the module's ``state_dict`` (so a routing slip inside the oracle
  -- the wrong sub-module's weights, the wrong mode -- fails);
* with two consecutive ops non-zero, the second must see the first one's
  output; the reversed order (or the second op reading the un-updated input)
  is a negative control that must differ.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd.pairformer import PairformerBlockHip
from bioemu2_amd.pairmixer import PairMixerLayerHip, PairMixerMSALayerHip
from tests._helpers import randomize_params, state

# Output projection(s) of every op, per composition: zeroing them makes that op's update exactly 0.
BLOCK_OUT = {
    "tri_mul_out": ["tri_mul_out.p_out.weight"],
    "tri_mul_in": ["tri_mul_in.p_out.weight"],
    "tri_att_start": ["tri_att_start.proj_o.weight"],
    "tri_att_end": ["tri_att_end.proj_o.weight"],
    "transition_z": ["transition_z.fc3.weight"],
    "attention_pair_bias": ["attention_pair_bias.proj_o.weight"],
    "transition_s": ["transition_s.fc3.weight"],
}
LAYER_OUT = {
    "tri_mul_out": ["tri_mul_out.p_out.weight"],
    "tri_mul_in": ["tri_mul_in.p_out.weight"],
    "transition_z": ["transition_z.fc3.weight"],
}
MSA_OUT = {
    "pair_weighted_averaging": ["pair_weighted_averaging.proj_o.weight"],
    "msa_transition": ["msa_transition.fc3.weight"],
    "outer_product_mean": ["outer_product_mean.proj_o.weight", "outer_product_mean.proj_o.bias"],
    "tri_mul_out": ["tri_mul_out.p_out.weight"],
    "tri_mul_in": ["tri_mul_in.p_out.weight"],
    "z_transition": ["z_transition.fc3.weight"],
}


def _sub(P: dict, prefix: str) -> dict:
    return {k[len(prefix) + 1:]: v for k, v in P.items() if k.split(".", 1)[0] == prefix}


def _only(P: dict, table: dict, keep: set[str]) -> dict:
    """P with the output projections of every op not in ``keep`` zeroed."""
    Q = dict(P)
    for op, keys in table.items():
        if op not in keep:
            for k in keys:
                Q[k] = torch.zeros_like(Q[k])
    return Q


# ----------------------------------------------------------------------------
# Pairformer block
# ----------------------------------------------------------------------------
N_BLK = 10


@pytest.fixture(scope="module")
def block_case():
    torch.manual_seed(0)
    P = state(randomize_params(PairformerBlockHip(), 11))
    g = torch.Generator().manual_seed(1)
    s = torch.randn(1, N_BLK, 384, generator=g)
    z = torch.randn(1, N_BLK, N_BLK, 128, generator=g)
    tok = torch.ones(1, N_BLK, dtype=torch.bool)
    tok[:, -2:] = False
    return P, s, z, tok, oracle.pair_mask_from_token_mask(tok)


def _blk_update(op: str, P: dict, s, z, tok, pm):
    """(new s, new z) after applying op alone to (s, z), from the per-op oracle functions."""
    Q = _sub(P, op)
    if op == "tri_mul_out":
        return s, z + oracle.trimul(z, pm, Q, "outgoing")
    if op == "tri_mul_in":
        return s, z + oracle.trimul(z, pm, Q, "incoming")
    if op == "tri_att_start":
        return s, z + oracle.triangle_attention(z, pm, Q, 4, starting=True)
    if op == "tri_att_end":
        return s, z + oracle.triangle_attention(z, pm, Q, 4, starting=False)
    if op == "transition_z":
        return s, z + oracle.transition(z, Q)
    if op == "attention_pair_bias":
        return s + oracle.attention_pair_bias(s, z, tok, Q, 16, tile_size=None), z
    if op == "transition_s":
        return s + oracle.transition(s, Q), z
    raise AssertionError(op)


def test_block_zero_updates_is_identity(block_case):
    P, s, z, tok, _ = block_case
    s2, z2 = oracle.pairformer_block(s, z, tok, _only(P, BLOCK_OUT, set()))
    assert torch.equal(s2, s) and torch.equal(z2, z)


@pytest.mark.parametrize("op", list(BLOCK_OUT))
def test_block_single_op(block_case, op):
    P, s, z, tok, pm = block_case
    Q = _only(P, BLOCK_OUT, {op})
    s2, z2 = oracle.pairformer_block(s, z, tok, Q)
    ws, wz = _blk_update(op, Q, s, z, tok, pm)
    assert torch.equal(s2, ws) and torch.equal(z2, wz)
    assert not (torch.equal(s2, s) and torch.equal(z2, z))  # the op does change something


@pytest.mark.parametrize(
    "first,second",
    [("tri_mul_out", "tri_mul_in"), ("tri_mul_in", "tri_att_start"), ("tri_att_start", "tri_att_end"),
     ("tri_att_end", "transition_z"), ("transition_z", "attention_pair_bias"),
     ("attention_pair_bias", "transition_s")],
)
def test_block_order(block_case, first, second):
    P, s, z, tok, pm = block_case
    Q = _only(P, BLOCK_OUT, {first, second})
    s2, z2 = oracle.pairformer_block(s, z, tok, Q)
    ws, wz = _blk_update(second, Q, *_blk_update(first, Q, s, z, tok, pm), tok, pm)
    assert torch.equal(s2, ws) and torch.equal(z2, wz)
    # Negative control: the reversed order gives a different result.
    rs, rz = _blk_update(first, Q, *_blk_update(second, Q, s, z, tok, pm), tok, pm)
    assert not (torch.allclose(rs, s2, atol=1e-4) and torch.allclose(rz, z2, atol=1e-4))


def test_block_starting_ending_not_interchangeable(block_case):
    P, s, z, tok, pm = block_case
    Q = _only(P, BLOCK_OUT, {"tri_att_start"})
    _, z2 = oracle.pairformer_block(s, z, tok, Q)
    swapped = z + oracle.triangle_attention(z, pm, _sub(Q, "tri_att_start"), 4, starting=False)
    assert not torch.allclose(z2, swapped, atol=1e-4)


# ----------------------------------------------------------------------------
# PairMixer layer (the reference trunk's layer)
# ----------------------------------------------------------------------------
@pytest.fixture(scope="module")
def layer_case():
    torch.manual_seed(0)
    P = state(randomize_params(PairMixerLayerHip(384, 128), 12))
    g = torch.Generator().manual_seed(2)
    n = 9
    s = torch.randn(1, n, 384, generator=g)
    z = torch.randn(1, n, n, 128, generator=g)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, -1:] = False
    return P, s, z, oracle.pair_mask_from_token_mask(tok)


def _layer_update(op, P, z, pm):
    Q = _sub(P, op)
    if op == "tri_mul_out":
        return z + oracle.trimul(z, pm, Q, "outgoing")
    if op == "tri_mul_in":
        return z + oracle.trimul(z, pm, Q, "incoming")
    return z + oracle.transition(z, Q)


def test_layer_zero_updates_is_identity(layer_case):
    P, s, z, pm = layer_case
    s2, z2 = oracle.pairmixer_layer(s, z, pm, _only(P, LAYER_OUT, set()))
    assert torch.equal(s2, s) and torch.equal(z2, z)


@pytest.mark.parametrize("op", list(LAYER_OUT))
def test_layer_single_op(layer_case, op):
    P, s, z, pm = layer_case
    Q = _only(P, LAYER_OUT, {op})
    s2, z2 = oracle.pairmixer_layer(s, z, pm, Q)
    assert torch.equal(s2, s) and torch.equal(z2, _layer_update(op, Q, z, pm))
    assert not torch.equal(z2, z)


@pytest.mark.parametrize("first,second", [("tri_mul_out", "tri_mul_in"), ("tri_mul_in", "transition_z")])
def test_layer_order(layer_case, first, second):
    P, s, z, pm = layer_case
    Q = _only(P, LAYER_OUT, {first, second})
    _, z2 = oracle.pairmixer_layer(s, z, pm, Q)
    assert torch.equal(z2, _layer_update(second, Q, _layer_update(first, Q, z, pm), pm))
    assert not torch.allclose(z2, _layer_update(first, Q, _layer_update(second, Q, z, pm), pm), atol=1e-4)


# ----------------------------------------------------------------------------
# PairMixer MSA layer
# ----------------------------------------------------------------------------
@pytest.fixture(scope="module")
def msa_case():
    torch.manual_seed(0)
    P = state(randomize_params(PairMixerMSALayerHip(384, 64, 128, 0.15, 0.25), 13))
    g = torch.Generator().manual_seed(3)
    n, S = 8, 5
    s = torch.randn(1, n, 384, generator=g)
    z = torch.randn(1, n, n, 128, generator=g)
    m = torch.randn(1, S, n, 64, generator=g)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, -1:] = False
    msa_mask = tok[:, None, :].expand(1, S, n).clone()
    msa_mask[:, -1] = False
    return P, s, z, m, oracle.pair_mask_from_token_mask(tok), msa_mask


def _msa_update(op, P, z, m, pm, msa_mask):
    """(new z, new m) after op alone."""
    Q = _sub(P, op)
    if op == "pair_weighted_averaging":
        return z, m + oracle.pair_weighted_averaging(m, z, pm, Q)
    if op == "msa_transition":
        return z, m + oracle.transition(m, Q)
    if op == "outer_product_mean":
        return z + oracle.outer_product_mean(m, msa_mask, Q), m
    if op == "tri_mul_out":
        return z + oracle.trimul(z, pm, Q, "outgoing"), m
    if op == "tri_mul_in":
        return z + oracle.trimul(z, pm, Q, "incoming"), m
    if op == "z_transition":
        return z + oracle.transition(z, Q), m
    raise AssertionError(op)


def test_msa_zero_updates_is_identity(msa_case):
    P, s, z, m, pm, mm = msa_case
    s2, z2, m2 = oracle.pairmixer_msa_layer(s, z, m, pm, mm, _only(P, MSA_OUT, set()))
    assert torch.equal(s2, s) and torch.equal(z2, z) and torch.equal(m2, m)


@pytest.mark.parametrize("op", list(MSA_OUT))
def test_msa_single_op(msa_case, op):
    P, s, z, m, pm, mm = msa_case
    Q = _only(P, MSA_OUT, {op})
    _, z2, m2 = oracle.pairmixer_msa_layer(s, z, m, pm, mm, Q)
    wz, wm = _msa_update(op, Q, z, m, pm, mm)
    assert torch.equal(z2, wz) and torch.equal(m2, wm)
    assert not (torch.equal(z2, z) and torch.equal(m2, m))


@pytest.mark.parametrize(
    "first,second",
    [("pair_weighted_averaging", "msa_transition"), ("msa_transition", "outer_product_mean"),
     ("pair_weighted_averaging", "outer_product_mean"), ("outer_product_mean", "tri_mul_out"),
     ("tri_mul_out", "tri_mul_in"), ("tri_mul_in", "z_transition")],
)
def test_msa_order(msa_case, first, second):
    P, s, z, m, pm, mm = msa_case
    Q = _only(P, MSA_OUT, {first, second})
    _, z2, m2 = oracle.pairmixer_msa_layer(s, z, m, pm, mm, Q)
    wz, wm = _msa_update(second, Q, *_msa_update(first, Q, z, m, pm, mm), pm, mm)
    assert torch.equal(z2, wz) and torch.equal(m2, wm)
    rz, rm = _msa_update(first, Q, *_msa_update(second, Q, z, m, pm, mm), pm, mm)
    assert not (torch.allclose(rz, z2, atol=1e-4) and torch.allclose(rm, m2, atol=1e-4))
