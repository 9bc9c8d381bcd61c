"""Host-side API of the drop-in modules (CPU only, no kernel launches).

Parameter names and shapes follow the reference's module definitions:
triangle_multiplication.py:71-76, attention_pair_bias.py:85-92,
outer_product_mean.py:37-39, transition.py:46-49,
pair_weighted_averaging.py:44-54 and modules/pairmixer.py:406-423 / :667-709;
``make()`` follows utils/strategy.py:13-50.
"""

from __future__ import annotations

import pytest
import torch

from bioemu2_amd.attention_pair_bias import AttentionPairBias, AttentionPairBiasSlidingWindow
from bioemu2_amd.glue import DistogramModule, PairwiseConditioning
from bioemu2_amd.outer_product_mean import REGISTRY as OPM_REGISTRY
from bioemu2_amd.outer_product_mean import OuterProductMeanHip
from bioemu2_amd.pair_weighted_averaging import PairWeightedAveraging
from bioemu2_amd.pairmixer import PairMixerLayerHip, PairMixerMSALayerHip
from bioemu2_amd.strategy import make
from bioemu2_amd.transition import Transition
from bioemu2_amd.triangle_attention import REGISTRY as TRIATT_REGISTRY
from bioemu2_amd.triangle_attention import TriangleAttentionEndingNodeHip, TriangleAttentionStartingNodeHip
from bioemu2_amd.triangle_multiplication import REGISTRY as TRIMUL_REGISTRY
from bioemu2_amd.triangle_multiplication import TriangleMultiplicationHip

C = 128

TRIMUL = {
    "norm_in.weight": (C,), "norm_in.bias": (C,), "p_in.weight": (2 * C, C), "g_in.weight": (2 * C, C),
    "norm_out.weight": (C,), "norm_out.bias": (C,), "p_out.weight": (C, C), "g_out.weight": (C, C),
}
TRANSITION_Z = {"norm.weight": (C,), "norm.bias": (C,), "fc1.weight": (4 * C, C), "fc2.weight": (4 * C, C),
                "fc3.weight": (C, 4 * C)}
TRANSITION_M = {"norm.weight": (64,), "norm.bias": (64,), "fc1.weight": (256, 64), "fc2.weight": (256, 64),
                "fc3.weight": (64, 256)}
PWA = {"norm_m.weight": (64,), "norm_m.bias": (64,), "norm_z.weight": (C,), "norm_z.bias": (C,),
       "proj_m.weight": (256, 64), "proj_g.weight": (256, 64), "proj_z.weight": (8, C), "proj_o.weight": (64, 256)}
OPM = {"norm.weight": (64,), "norm.bias": (64,), "proj_ab.weight": (64, 64), "proj_o.weight": (C, 1024),
       "proj_o.bias": (C,)}


def _shapes(module: torch.nn.Module) -> dict[str, tuple[int, ...]]:
    return {k: tuple(v.shape) for k, v in module.state_dict().items()}


def _prefixed(prefix: str, d: dict) -> dict:
    return {f"{prefix}.{k}": v for k, v in d.items()}


def test_trimul_state_dict_matches_reference_names():
    for mode in ("outgoing", "incoming"):
        assert _shapes(TriangleMultiplicationHip(dim=C, mode=mode)) == TRIMUL


def test_apb_state_dict_matches_reference_names():
    got = _shapes(AttentionPairBias(384, C, 16, initial_norm=True, use_bias_in_layer_norm=True))
    assert got == {"norm_s.weight": (384,), "norm_s.bias": (384,), "proj_qkv.weight": (3 * 384, 384),
                   "proj_q_bias": (384,), "proj_g.weight": (384, 384), "norm_z.weight": (C,),
                   "norm_z.bias": (C,), "proj_z.weight": (16, C), "proj_o.weight": (384, 384)}
    got = _shapes(AttentionPairBias(384, C, 16, initial_norm=False, use_bias_in_layer_norm=False))
    assert "norm_s.weight" not in got and "norm_z.bias" not in got


def test_opm_transition_pwa_state_dicts():
    assert _shapes(OuterProductMeanHip(64, 32, C)) == OPM
    assert _shapes(Transition(C, 4 * C)) == TRANSITION_Z
    assert set(_shapes(Transition(C, 4 * C, use_norm=False))) == {"fc1.weight", "fc2.weight", "fc3.weight"}
    assert _shapes(PairWeightedAveraging(64, C, 32, 8)) == PWA
    assert "norm_z.bias" not in _shapes(PairWeightedAveraging(64, C, 32, 8, use_bias_in_layer_norm=False))


def test_sliding_window_and_glue_state_dicts():
    swa = _shapes(AttentionPairBiasSlidingWindow(128, 16, 4))
    assert swa == {"norm_s.weight": (128,), "norm_s.bias": (128,), "proj_qkv.weight": (384, 128),
                   "proj_q_bias": (128,), "proj_g.weight": (128, 128), "norm_z.weight": (16,),
                   "proj_z.weight": (4, 16), "proj_o.weight": (128, 128)}
    assert "norm_s.weight" not in _shapes(AttentionPairBiasSlidingWindow(128, 16, 4, initial_norm=False))
    assert _shapes(DistogramModule(C, 64)) == {"distogram.weight": (64, C), "distogram.bias": (64,)}
    tz = {k: v for k, v in TRANSITION_Z.items()}
    tz.update({"fc1.weight": (2 * C, C), "fc2.weight": (2 * C, C), "fc3.weight": (C, 2 * C)})
    want = {"dim_pairwise_init_proj.0.weight": (2 * C,), "dim_pairwise_init_proj.0.bias": (2 * C,),
            "dim_pairwise_init_proj.1.weight": (C, 2 * C), **_prefixed("transitions.0", tz),
            **_prefixed("transitions.1", tz)}
    assert _shapes(PairwiseConditioning(C, C)) == want


def test_pairmixer_layer_state_dict_and_variants():
    """As the reference's test_full_and_cueq_have_same_state_dict_keys (tests/biomoa/modules/test_pairmixer.py)."""
    want = {**_prefixed("tri_mul_out", TRIMUL), **_prefixed("tri_mul_in", TRIMUL),
            **_prefixed("transition_z", TRANSITION_Z)}
    for variant in ("full", "cueq", "cueq_tiled"):
        assert _shapes(PairMixerLayerHip(token_s=384, token_z=C, trimul_variant=variant)) == want
    with pytest.raises(ValueError, match="Unknown variant"):
        PairMixerLayerHip(token_s=384, token_z=C, trimul_variant="bogus")


def test_pairmixer_msa_layer_state_dict():
    want = {**_prefixed("msa_transition", TRANSITION_M), **_prefixed("pair_weighted_averaging", PWA),
            **_prefixed("tri_mul_out", TRIMUL), **_prefixed("tri_mul_in", TRIMUL),
            **_prefixed("z_transition", TRANSITION_Z), **_prefixed("outer_product_mean", OPM)}
    for opm in ("vanilla", "triton_memory_saving"):
        assert _shapes(PairMixerMSALayerHip(384, 64, C, 0.15, 0.25, opm_variant=opm)) == want


def test_state_dict_round_trip_between_instances():
    a = PairMixerMSALayerHip(384, 64, C, 0.15, 0.25)
    for p in a.parameters():
        torch.nn.init.normal_(p)
    b = PairMixerMSALayerHip(384, 64, C, 0.15, 0.25, trimul_variant="full")
    b.load_state_dict(a.state_dict())
    for k, v in a.state_dict().items():
        assert torch.equal(v, b.state_dict()[k])


def test_make_contract():
    m = make(TRIMUL_REGISTRY, "cueq", dim=C, mode="incoming", matmul_precision="highest")
    assert isinstance(m, TriangleMultiplicationHip) and m.mode == "incoming"
    assert isinstance(make(OPM_REGISTRY, "vanilla", c_in=64, c_hidden=32, c_out=C), OuterProductMeanHip)
    assert isinstance(make(TRIATT_REGISTRY, "hip", starting=True, c_z=C, num_heads=4),
                      TriangleAttentionStartingNodeHip)
    assert isinstance(make(TRIATT_REGISTRY, "hip", starting=False, c_z=C, num_heads=4),
                      TriangleAttentionEndingNodeHip)
    with pytest.raises(ValueError, match="Unknown variant"):
        make(OPM_REGISTRY, "nope", c_in=64, c_hidden=32, c_out=C)


def test_cpu_tensors_are_rejected_without_fallback():
    """The product path has no CPU fallback: every module raises on host tensors."""
    z = torch.randn(1, 8, 8, C)
    pm = torch.ones(1, 8, 8, dtype=torch.bool)
    m = torch.randn(1, 4, 8, 64)
    with pytest.raises(RuntimeError, match="no CPU path"):
        TriangleMultiplicationHip(dim=C)(z, pm)
    with pytest.raises(RuntimeError, match="no CPU path"):
        Transition(C, 4 * C)(z)
    with pytest.raises(RuntimeError, match="no CPU path"):
        PairWeightedAveraging(64, C, 32, 8)(m, z, pm)
    with pytest.raises(RuntimeError, match="no CPU path"):
        PairMixerLayerHip(384, C)(None, z, pm)
    with pytest.raises(RuntimeError, match="no CPU path"):
        PairMixerMSALayerHip(384, 64, C, 0.15, 0.25)(None, z, m, pm, torch.ones(1, 4, 8, dtype=torch.bool))


def test_transition_out_dim_matches_reference_layout():
    """Transition(dim, hidden, out_dim, use_norm=False) as the denoiser's mixers build it (diffusion.py:623-634):
    no norm.* keys, fc3 maps hidden -> out_dim (transition.py:34-50)."""
    t = Transition(512, 1024, out_dim=128, use_norm=False)
    sd = t.state_dict()
    assert sorted(sd) == ["fc1.weight", "fc2.weight", "fc3.weight"]
    assert sd["fc1.weight"].shape == (1024, 512) and sd["fc3.weight"].shape == (128, 1024)
