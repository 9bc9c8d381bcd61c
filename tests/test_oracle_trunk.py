"""Pins the oracle's PairMixer trunk functions (CPU).

``oracle.ln_linear`` (recycling updates, pairmixer.py:281-282), ``oracle.msa_embed`` (pairmixer.py:591-599),
``oracle.pairmixer_module`` (:352-370), ``oracle.pairmixer_msa_module`` (:553-611) and
``oracle.pairmixer_trunk`` (:275-296).  The layers themselves are pinned elsewhere
(test_oracle_compositions.py); here:

* ``ln_linear``: brute-force numpy loops; zero weight returns base exactly; an identity weight with a
  unit LayerNorm returns base + a row of mean 0 and variance 1.
* ``msa_embed``: brute-force numpy loops; a one-hot MSA row selects exactly that column of ``msa_proj``;
  the concatenation order (msa, has_deletion, deletion_value, msa_paired) is pinned by planting distinct
  values in each feature and reading them back through an identity-like weight.
* ``pairmixer_module``: 0 blocks is the identity; 2 blocks equal layer 0 then layer 1 (the reversed order
  is a negative control that must differ).
* ``pairmixer_msa_module``: 1 block equals msa_embed + the MSA layer (with s = None and the pair mask).
* ``pairmixer_trunk``: with 0 PairMixer blocks and 0 MSA blocks, one pass is the two recycling updates of
  zero; a second pass recycles the first pass's output (closed forms from ``ln_linear``).
* ``pairmixer_uncond``: brute-force numpy loops; a zero ``fc3`` returns z_init (and s_init) exactly; a
  ``z_norm`` with zero weight feeds every row the constant ``z_norm.bias``, whose own LayerNorm is the
  transition norm's bias, so every row gains the same closed-form vector; skipping ``z_norm`` (a negative
  control) changes the result.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from bioemu2_amd.pairmixer import NUM_TOKENS, PairMixerModuleHip, PairMixerMSAModuleHip, PairMixerTrunkHip
from tests._helpers import np_ln, randomize_params, state


def _ln_params(prefix: str, width: int, g: torch.Generator, w: torch.Tensor) -> dict:
    return {f"{prefix}_norm.weight": 1 + 0.1 * torch.randn(width, generator=g),
            f"{prefix}_norm.bias": 0.1 * torch.randn(width, generator=g), f"{prefix}_recycle.weight": w}


def test_ln_linear_brute_force_and_special_cases():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 5, 16, generator=g)
    base = torch.randn(2, 5, 16, generator=g)
    P = _ln_params("z", 16, g, torch.randn(16, 16, generator=g) / 4)
    got = oracle.ln_linear(x, base, P, "z_norm", "z_recycle")
    w, lw, lb = (P[k].double().numpy() for k in ("z_recycle.weight", "z_norm.weight", "z_norm.bias"))
    for b in range(2):
        for t in range(5):
            want = base[b, t].double().numpy() + w @ np_ln(x[b, t].double().numpy(), lw, lb)
            np.testing.assert_allclose(got[b, t].numpy(), want, rtol=1e-5, atol=1e-5)
    Z = dict(P, **{"z_recycle.weight": torch.zeros(16, 16)})
    assert torch.equal(oracle.ln_linear(x, base, Z, "z_norm", "z_recycle"), base)
    unit = {"z_norm.weight": torch.ones(16), "z_norm.bias": torch.zeros(16), "z_recycle.weight": torch.eye(16)}
    d = oracle.ln_linear(x, base, unit, "z_norm", "z_recycle") - base
    torch.testing.assert_close(d.mean(-1), torch.zeros(2, 5), atol=1e-5, rtol=0)
    torch.testing.assert_close(d.var(-1, unbiased=False), torch.ones(2, 5), atol=1e-3, rtol=0)


def _msa_feats(B, R, T, g, paired=True):
    tok = torch.randint(0, NUM_TOKENS, (B, R, T), generator=g)
    return {
        "msa": torch.nn.functional.one_hot(tok, NUM_TOKENS).float(),
        "has_deletion": (torch.rand(B, R, T, generator=g) < 0.3).float(),
        "deletion_value": torch.rand(B, R, T, generator=g),
        "msa_paired": (torch.rand(B, R, T, generator=g) < 0.5).float() if paired else None,
        "msa_mask": (torch.rand(B, R, T, generator=g) > 0.2),
        "tok": tok,
    }


def test_msa_embed_brute_force_one_hot_and_feature_order():
    g = torch.Generator().manual_seed(1)
    B, R, T, E, C = 1, 3, 4, 10, 64
    f = _msa_feats(B, R, T, g)
    emb = torch.randn(B, T, E, generator=g)
    P = {"msa_proj.weight": torch.randn(C, NUM_TOKENS + 3, generator=g), "s_proj.weight": torch.randn(C, E, generator=g)}
    got = oracle.msa_embed(f["msa"], f["has_deletion"], f["deletion_value"], f["msa_paired"], emb, P)
    wm, ws = P["msa_proj.weight"].double().numpy(), P["s_proj.weight"].double().numpy()
    for r in range(R):
        for t in range(T):
            feat = np.concatenate([f["msa"][0, r, t].double().numpy(),
                                   [f["has_deletion"][0, r, t].item(), f["deletion_value"][0, r, t].item(),
                                    f["msa_paired"][0, r, t].item()]])
            want = wm @ feat + ws @ emb[0, t].double().numpy()
            np.testing.assert_allclose(got[0, r, t].numpy(), want, rtol=1e-5, atol=1e-5)
            # one-hot row: exactly the token's weight column plus the s_proj row
            col = wm[:, f["tok"][0, r, t]] + wm[:, NUM_TOKENS] * feat[NUM_TOKENS] + \
                wm[:, NUM_TOKENS + 1] * feat[NUM_TOKENS + 1] + wm[:, NUM_TOKENS + 2] * feat[NUM_TOKENS + 2]
            np.testing.assert_allclose(got[0, r, t].numpy(), col + ws @ emb[0, t].double().numpy(), rtol=1e-5,
                                       atol=1e-5)
    # feature order: output channel k reads feature k only
    eye = torch.zeros(C, NUM_TOKENS + 3)
    eye[:NUM_TOKENS + 3, :] = torch.eye(NUM_TOKENS + 3)
    Q = {"msa_proj.weight": eye, "s_proj.weight": torch.zeros(C, E)}
    m = oracle.msa_embed(f["msa"], f["has_deletion"], f["deletion_value"], f["msa_paired"], emb, Q)
    assert torch.equal(m[..., :NUM_TOKENS], f["msa"])
    assert torch.equal(m[..., NUM_TOKENS], f["has_deletion"])
    assert torch.equal(m[..., NUM_TOKENS + 1], f["deletion_value"])
    assert torch.equal(m[..., NUM_TOKENS + 2], f["msa_paired"])
    # without the paired feature the weight has NUM_TOKENS + 2 columns
    m2 = oracle.msa_embed(f["msa"], f["has_deletion"], f["deletion_value"], None, emb,
                          {"msa_proj.weight": eye[:, :NUM_TOKENS + 2], "s_proj.weight": torch.zeros(C, E)})
    assert torch.equal(m2[..., NUM_TOKENS + 1], f["deletion_value"])


def _pm_case(n=8, blocks=2, seed=3):
    torch.manual_seed(0)
    P = state(randomize_params(PairMixerModuleHip(384, 128, blocks), seed))
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(1, n, 384, generator=g)
    z = torch.randn(1, n, n, 128, generator=g)
    tok = torch.ones(1, n, dtype=torch.bool)
    tok[:, -2:] = False
    return P, s, z, oracle.pair_mask_from_token_mask(tok)


def _sub(P: dict, prefix: str) -> dict:
    return {k[len(prefix) + 1:]: v for k, v in P.items() if k.startswith(prefix + ".")}


def test_pairmixer_module_is_the_layers_in_order():
    P, s, z, pm = _pm_case()
    s0, z0 = oracle.pairmixer_module(s, z, pm, P, 0)
    assert torch.equal(s0, s) and torch.equal(z0, z)
    _, got = oracle.pairmixer_module(s, z, pm, P, 2)
    _, z1 = oracle.pairmixer_layer(s, z, pm, _sub(P, "layers.0"))
    _, want = oracle.pairmixer_layer(s, z1, pm, _sub(P, "layers.1"))
    assert torch.equal(got, want)
    _, r1 = oracle.pairmixer_layer(s, z, pm, _sub(P, "layers.1"))
    _, rev = oracle.pairmixer_layer(s, r1, pm, _sub(P, "layers.0"))
    assert (rev - got).abs().max() > 1e-3


def test_pairmixer_msa_module_is_embed_then_layers():
    torch.manual_seed(0)
    mod = PairMixerMSAModuleHip(384, 64, 128, 20, msa_blocks=1, msa_dropout=0.15, z_dropout=0.25,
                                use_paired_feature=True)
    P = state(randomize_params(mod, 5))
    g = torch.Generator().manual_seed(6)
    B, R, T = 1, 5, 7
    f = _msa_feats(B, R, T, g)
    emb = torch.randn(B, T, 20, generator=g)
    z = torch.randn(B, T, T, 128, generator=g)
    tok = torch.ones(B, T, dtype=torch.bool)
    tok[:, -1] = False
    got = oracle.pairmixer_msa_module(z, emb, f, tok, P, 1)
    m = oracle.msa_embed(f["msa"], f["has_deletion"], f["deletion_value"], f["msa_paired"], emb, P)
    _, want, _ = oracle.pairmixer_msa_layer(None, z, m, oracle.pair_mask_from_token_mask(tok), f["msa_mask"],
                                            _sub(P, "layers.0"))
    assert torch.equal(got, want)


def test_pairmixer_trunk_recycling_closed_form():
    torch.manual_seed(0)
    mod = PairMixerTrunkHip(32, 128, 20, msa_blocks=0, num_blocks=0)
    P = state(randomize_params(mod, 8))
    g = torch.Generator().manual_seed(9)
    B, R, T = 1, 3, 6
    f = _msa_feats(B, R, T, g)
    f["token_pad_mask"] = torch.ones(B, T, dtype=torch.bool)
    s_init, z_init = torch.randn(B, T, 32, generator=g), torch.randn(B, T, T, 128, generator=g)
    emb = torch.randn(B, T, 20, generator=g)
    s1, z1 = oracle.pairmixer_trunk(s_init, z_init, emb, f, P, 0, 0, num_steps_recycle=0)
    assert torch.equal(s1, oracle.ln_linear(torch.zeros_like(s_init), s_init, P, "s_norm", "s_recycle"))
    assert torch.equal(z1, oracle.ln_linear(torch.zeros_like(z_init), z_init, P, "z_norm", "z_recycle"))
    # zero input through LayerNorm is its bias: one pass adds W beta to every row
    torch.testing.assert_close(s1, s_init + P["s_norm.bias"] @ P["s_recycle.weight"].T, rtol=1e-6, atol=1e-6)
    s2, z2 = oracle.pairmixer_trunk(s_init, z_init, emb, f, P, 0, 0, num_steps_recycle=1)
    assert torch.equal(s2, oracle.ln_linear(s1, s_init, P, "s_norm", "s_recycle"))
    assert torch.equal(z2, oracle.ln_linear(z1, z_init, P, "z_norm", "z_recycle"))


def test_trunk_modules_state_dict_layout():
    """Keys as the reference's modules define them (pairmixer.py:186-191, :527-532, :334-349)."""
    t = PairMixerTrunkHip(384, 128, 455, msa_blocks=2, num_blocks=3)
    sd = {k: tuple(v.shape) for k, v in t.state_dict().items()}
    assert sd["s_recycle.weight"] == (384, 384) and sd["z_recycle.weight"] == (128, 128)
    assert sd["s_norm.bias"] == (384,) and sd["z_norm.weight"] == (128,)
    assert sd["msa_module.s_proj.weight"] == (64, 455)
    assert sd["msa_module.msa_proj.weight"] == (64, NUM_TOKENS + 3)   # use_paired_feature=True by default
    assert {k.split(".")[2] for k in sd if k.startswith("pairmixer_module.layers.")} == {"0", "1", "2"}
    assert {k.split(".")[2] for k in sd if k.startswith("msa_module.layers.")} == {"0", "1"}
    assert "pairmixer_module.layers.2.tri_mul_in.p_out.weight" in sd
    assert "msa_module.layers.1.outer_product_mean.proj_o.bias" in sd


def _np_transition(x, P, prefix):
    w1, w2, w3 = (P[f"{prefix}.fc{i}.weight"].double().numpy() for i in (1, 2, 3))
    xn = np_ln(x, P[f"{prefix}.norm.weight"].double().numpy(), P[f"{prefix}.norm.bias"].double().numpy())
    a = w1 @ xn
    return w3 @ (a / (1 + np.exp(-a)) * (w2 @ xn))


def test_pairmixer_uncond_closed_forms():
    torch.manual_seed(0)
    mod = PairMixerTrunkHip(32, 128, 20, msa_blocks=0, num_blocks=0, use_unconditional_branch=True)
    P = state(randomize_params(mod, 3))
    g = torch.Generator().manual_seed(5)
    s_init, z_init = torch.randn(1, 5, 32, generator=g), torch.randn(1, 5, 5, 128, generator=g) * 2
    s, z = oracle.pairmixer_uncond(s_init, z_init, P)
    assert torch.equal(s, s_init)
    zw, zb = P["z_norm.weight"].double().numpy(), P["z_norm.bias"].double().numpy()
    for i in range(5):
        for j in range(5):
            row = z_init[0, i, j].double().numpy()
            want = row + _np_transition(np_ln(row, zw, zb), P, "uncond_transition")
            np.testing.assert_allclose(z[0, i, j].numpy(), want, rtol=1e-5, atol=1e-5)
    Z = dict(P, **{"uncond_transition.fc3.weight": torch.zeros(128, 512)})
    assert torch.equal(oracle.pairmixer_uncond(s_init, z_init, Z)[1], z_init)
    # z_norm with zero weight and a constant bias makes every transition input the row (0.7, ..., 0.7), whose
    # LayerNorm is exactly the transition norm's bias: every row gains W3 (silu(W1 b) * (W2 b)), b that bias
    C = dict(P, **{"z_norm.weight": torch.zeros(128), "z_norm.bias": torch.full((128,), 0.7)})
    tb = P["uncond_transition.norm.bias"].double().numpy()
    w1, w2, w3 = (P[f"uncond_transition.fc{i}.weight"].double().numpy() for i in (1, 2, 3))
    a = w1 @ tb
    const = w3 @ (a / (1 + np.exp(-a)) * (w2 @ tb))
    zc = oracle.pairmixer_uncond(s_init, z_init, C)[1]
    np.testing.assert_allclose((zc - z_init).reshape(-1, 128).numpy(), np.broadcast_to(const, (25, 128)),
                               rtol=1e-4, atol=1e-4)
    skip = z_init + oracle.transition(z_init, {k[len("uncond_transition."):]: v for k, v in P.items()
                                               if k.startswith("uncond_transition.")})
    assert (skip - z).abs().max() > 1e-2


def test_trunk_unconditional_state_dict_layout():
    """uncond_transition = Transition(token_z, 4 token_z) exists only with use_unconditional_branch (:193-200)."""
    sd = PairMixerTrunkHip(64, 128, 20, msa_blocks=0, num_blocks=0, use_unconditional_branch=True).state_dict()
    assert tuple(sd["uncond_transition.fc1.weight"].shape) == (512, 128)
    assert tuple(sd["uncond_transition.fc3.weight"].shape) == (128, 512)
    assert tuple(sd["uncond_transition.norm.weight"].shape) == (128,)
    plain = PairMixerTrunkHip(64, 128, 20, msa_blocks=0, num_blocks=0).state_dict()
    assert not any(k.startswith("uncond_transition.") for k in plain)
