"""``integration.install()`` against a stub package laid out like the reference (CPU only).

The stub's modules bind their ops the way the reference's do, with ``from <pkg>.biomoa.ops.X import Y`` at
import time (modules/transformer.py:22-23, modules/pairmixer.py:11-18, modules/diffusion.py:26,
models/score_model.py:14), resolve TriMul and OPM through registries and ``make()``
(ops/triangle_multiplication.py:348-352, ops/outer_product_mean.py:155-158, utils/strategy.py:13-50), and
construct them with the reference's kwargs (transformer.py:97-115, :311; pairmixer.py:667-709;
diffusion.py:151-157, :623-634; score_model.py:213). After ``install()`` every construction yields the HIP
class; ``undo()`` restores the stubs.
"""

from __future__ import annotations

import importlib
import sys
import textwrap

import pytest

from bioemu2_amd import attention_pair_bias as hip_apb
from bioemu2_amd import glue as hip_glue
from bioemu2_amd import integration
from bioemu2_amd import outer_product_mean as hip_opm
from bioemu2_amd import pair_weighted_averaging as hip_pwa
from bioemu2_amd import pairmixer as hip_pm
from bioemu2_amd import transition as hip_tr
from bioemu2_amd import triangle_multiplication as hip_tm

PKG = "refstub_bioemu2"


def _src(*parts: str) -> str:
    """Join source fragments, each dedented on its own."""
    return "\n".join(textwrap.dedent(part) for part in parts)


_STUB_CLASS = """
class {name}(nn.Module):
    def __init__(self, *args, **kwargs):
        super().__init__()
        self.args, self.kwargs = args, kwargs
"""

FILES = {
    "biomoa/ops/attention_pair_bias.py": "import torch.nn as nn\n" + _STUB_CLASS.format(name="AttentionPairBias")
    + _STUB_CLASS.format(name="AttentionPairBiasSlidingWindow"),
    "biomoa/ops/transition.py": "import torch.nn as nn\n" + _STUB_CLASS.format(name="Transition"),
    "biomoa/ops/pair_weighted_averaging.py": "import torch.nn as nn\n"
    + _STUB_CLASS.format(name="PairWeightedAveraging"),
    "biomoa/ops/triangle_multiplication.py": _src("""
        from enum import Enum
        import torch.nn as nn

        class TriMulVariant(str, Enum):
            FULL = "full"
            CUEQ = "cueq"
            CUEQ_TILED = "cueq_tiled"
        """, _STUB_CLASS.format(name="TriangleMultiplicationFull"),
        _STUB_CLASS.format(name="TriangleMultiplicationCueq"), _STUB_CLASS.format(name="TriangleMultiplicationCueqTiled"),
        """
        REGISTRY = {
            TriMulVariant.FULL: (__name__, "TriangleMultiplicationFull"),
            TriMulVariant.CUEQ: (__name__, "TriangleMultiplicationCueq"),
            TriMulVariant.CUEQ_TILED: (__name__, "TriangleMultiplicationCueqTiled"),
        }
        """),
    "biomoa/ops/outer_product_mean.py": _src("""
        from enum import Enum
        import torch.nn as nn

        class OPMVariant(str, Enum):
            VANILLA = "vanilla"
            TRITON_MEMORY_SAVING = "triton_memory_saving"
        """, _STUB_CLASS.format(name="OuterProductMeanVanilla"),
        _STUB_CLASS.format(name="OuterProductMeanTritonMemorySaving"), """
        REGISTRY = {
            OPMVariant.VANILLA: (__name__, "OuterProductMeanVanilla"),
            OPMVariant.TRITON_MEMORY_SAVING: (__name__, "OuterProductMeanTritonMemorySaving"),
        }
        """),
    "biomoa/utils/strategy.py": "from bioemu2_amd.strategy import make  # noqa: F401\n",
    "biomoa/modules/transformer.py": """
        import torch.nn as nn
        from {pkg}.biomoa.ops.attention_pair_bias import AttentionPairBias, AttentionPairBiasSlidingWindow
        from {pkg}.biomoa.ops.transition import Transition

        class AttentionLayer(nn.Module):
            def __init__(self, sliding=False):
                super().__init__()
                if sliding:
                    self.pair_bias_attn = AttentionPairBiasSlidingWindow(
                        c_s=128, c_z=16, num_heads=4, window_queries=32, window_keys=128,
                        initial_norm=False, zero_init_output=True)
                else:
                    self.pair_bias_attn = AttentionPairBias(
                        c_s=384, c_z=128, num_heads=16, initial_norm=False, zero_init_output=True, tile_size=512)
                self.transition = Transition(dim=384, hidden=768, use_norm=False)
        """,
    "biomoa/modules/pairmixer.py": """
        import torch.nn as nn
        from {pkg}.biomoa.ops.outer_product_mean import REGISTRY as OPM_REGISTRY
        from {pkg}.biomoa.ops.outer_product_mean import OPMVariant
        from {pkg}.biomoa.ops.pair_weighted_averaging import PairWeightedAveraging
        from {pkg}.biomoa.ops.transition import Transition
        from {pkg}.biomoa.ops.triangle_multiplication import REGISTRY as TRIMUL_REGISTRY
        from {pkg}.biomoa.ops.triangle_multiplication import TriMulVariant
        from {pkg}.biomoa.utils.strategy import make

        class PairMixerLayer(nn.Module):
            def __init__(self, token_s, token_z, dropout=0.25, trimul_variant="cueq", trimul_tile_size=None,
                         transition_chunk_size=None, trimul_matmul_precision=None):
                super().__init__()
                v = TriMulVariant(trimul_variant)
                self.tri_mul_out = make(TRIMUL_REGISTRY, v, mode="outgoing", dim=token_z,
                                        tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
                self.tri_mul_in = make(TRIMUL_REGISTRY, v, mode="incoming", dim=token_z,
                                       tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
                self.transition_z = Transition(dim=token_z, hidden=token_z * 4, chunk_size=transition_chunk_size)

        class PairMixerMSALayer(nn.Module):
            def __init__(self, token_s, msa_s, token_z, msa_dropout, z_dropout, trimul_variant="cueq",
                         trimul_tile_size=None, transition_chunk_size=None, opm_variant="vanilla",
                         opm_tile_size=None, opm_matmul_precision=None, trimul_matmul_precision=None):
                super().__init__()
                self.msa_transition = Transition(dim=msa_s, hidden=msa_s * 4, chunk_size=transition_chunk_size)
                self.pair_weighted_averaging = PairWeightedAveraging(c_m=msa_s, c_z=token_z, c_h=32, num_heads=8)
                v = TriMulVariant(trimul_variant)
                self.tri_mul_out = make(TRIMUL_REGISTRY, v, mode="outgoing", dim=token_z,
                                        tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
                self.tri_mul_in = make(TRIMUL_REGISTRY, v, mode="incoming", dim=token_z,
                                       tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
                self.z_transition = Transition(dim=token_z, hidden=token_z * 4, chunk_size=transition_chunk_size)
                self.outer_product_mean = make(OPM_REGISTRY, OPMVariant(opm_variant), c_in=msa_s, c_hidden=32,
                                               c_out=token_z, tile_size=opm_tile_size,
                                               matmul_precision=opm_matmul_precision)

        class PairMixerModule(nn.Module):
            def __init__(self, num_layers=2, trimul_variant="cueq"):
                super().__init__()
                self.layers = nn.ModuleList(
                    [PairMixerLayer(384, 128, trimul_variant=trimul_variant) for _ in range(num_layers)])
                self.msa_layer = PairMixerMSALayer(384, 64, 128, 0.15, 0.25, trimul_variant=trimul_variant)
        """,
    "biomoa/modules/embedders.py": "import torch.nn as nn\n" + _STUB_CLASS.format(name="DistogramModule"),
    "biomoa/modules/diffusion.py": _src("""
        import torch.nn as nn
        from {pkg}.biomoa.ops.transition import Transition

        class DiffusionConditioning(nn.Module):
            def __init__(self):
                super().__init__()
                self.pairwise_conditioner = PairwiseConditioning(
                    token_z=128, a_z=128, dim_token_rel_pos_feats=128, num_transitions=2,
                    transition_chunk_size=None)

        class AtomTokenMixer(nn.Module):
            def __init__(self, a_s=384, atom_s=128, transition_expansion_factor=2):
                super().__init__()
                self.s_to_q_mixer = Transition(dim=a_s + atom_s, hidden=transition_expansion_factor * (a_s + atom_s),
                                               out_dim=atom_s, use_norm=False)
                self.q_to_s_mixer = Transition(dim=a_s + atom_s, hidden=transition_expansion_factor * (a_s + atom_s),
                                               out_dim=a_s, use_norm=False)
        """, _STUB_CLASS.format(name="PairwiseConditioning")),
    "biomoa/models/score_model.py": """
        import torch.nn as nn
        from {pkg}.biomoa.modules.embedders import DistogramModule

        class ScoreModel(nn.Module):
            def __init__(self, token_z=128, num_bins_distogram=64):
                super().__init__()
                self.distogram_module = DistogramModule(token_z, num_bins_distogram)
        """,
}


@pytest.fixture
def ref(tmp_path, monkeypatch):
    """Write the stub package, import it fresh, and drop it from ``sys.modules`` afterwards."""
    for d in ("", "biomoa", "biomoa/ops", "biomoa/modules", "biomoa/models", "biomoa/utils"):
        p = tmp_path / PKG / d
        p.mkdir(parents=True, exist_ok=True)
        (p / "__init__.py").write_text("")
    for rel, text in FILES.items():
        (tmp_path / PKG / rel).write_text(textwrap.dedent(text).replace("{pkg}", PKG))
    monkeypatch.syspath_prepend(str(tmp_path))
    importlib.invalidate_caches()
    mods = {name: importlib.import_module(f"{PKG}.biomoa.{name}")
            for name in ("modules.transformer", "modules.pairmixer", "modules.diffusion", "models.score_model",
                         "ops.triangle_multiplication", "ops.outer_product_mean")}
    yield mods
    for name in [m for m in sys.modules if m == PKG or m.startswith(PKG + ".")]:
        del sys.modules[name]


def _types(mods):
    """Construct every caller the way the reference does and collect the classes it got."""
    tf, pm, dif, sm = (mods[k] for k in ("modules.transformer", "modules.pairmixer", "modules.diffusion",
                                         "models.score_model"))
    att, swa = tf.AttentionLayer(), tf.AttentionLayer(sliding=True)
    msa = pm.PairMixerMSALayer(384, 64, 128, 0.15, 0.25, trimul_variant="cueq_tiled",
                               opm_variant="triton_memory_saving", opm_matmul_precision="highest")
    layer = pm.PairMixerLayer(384, 128, trimul_variant="cueq", trimul_matmul_precision="highest")
    mixer = dif.AtomTokenMixer()
    return {
        "apb": type(att.pair_bias_attn), "swa": type(swa.pair_bias_attn), "token_transition": type(att.transition),
        "trimul_out": type(layer.tri_mul_out), "trimul_in": type(layer.tri_mul_in),
        "z_transition": type(layer.transition_z), "msa_transition": type(msa.msa_transition),
        "pwa": type(msa.pair_weighted_averaging), "trimul_tiled": type(msa.tri_mul_out),
        "opm": type(msa.outer_product_mean), "mixer": type(mixer.s_to_q_mixer),
        "pair_cond": type(dif.DiffusionConditioning().pairwise_conditioner),
        "distogram": type(sm.ScoreModel().distogram_module),
        "trimul_full": type(pm.PairMixerLayer(384, 128, trimul_variant="full").tri_mul_out),
    }


HIP = {
    "apb": hip_apb.AttentionPairBias, "swa": hip_apb.AttentionPairBiasSlidingWindow,
    "token_transition": hip_tr.Transition, "trimul_out": hip_tm.TriangleMultiplicationHip,
    "trimul_in": hip_tm.TriangleMultiplicationHip, "z_transition": hip_tr.Transition,
    "msa_transition": hip_tr.Transition, "pwa": hip_pwa.PairWeightedAveraging,
    "trimul_tiled": hip_tm.TriangleMultiplicationHip, "opm": hip_opm.OuterProductMeanHip,
    "mixer": hip_tr.Transition, "pair_cond": hip_glue.PairwiseConditioning,
    "distogram": hip_glue.DistogramModule,
}


def test_install_binds_hip_classes_where_the_callers_import_them(ref):
    before = _types(ref)
    assert all(t.__module__.startswith(PKG) for t in before.values())
    inst = integration.install(PKG)
    after = _types(ref)
    for key, cls in HIP.items():
        assert after[key] is cls, key
    assert after["trimul_full"] is before["trimul_full"]      # the eager variant stays the reference's
    layer = ref["modules.pairmixer"].PairMixerLayer(384, 128)
    assert layer.tri_mul_in.mode == "incoming" and layer.tri_mul_out.mode == "outgoing"
    mixer = ref["modules.diffusion"].AtomTokenMixer()
    assert mixer.s_to_q_mixer.fc3.weight.shape == (128, 1024) and mixer.q_to_s_mixer.out_dim == 384
    assert "norm.weight" not in mixer.s_to_q_mixer.state_dict()
    inst.undo()
    assert _types(ref) == before


def test_install_full_variant_and_whole_layers(ref):
    pm = ref["modules.pairmixer"]
    with integration.install(PKG, trimul_variants=("full", "cueq"), whole_layers=True):
        assert type(pm.PairMixerLayer(384, 128, trimul_variant="full").tri_mul_out) is hip_tm.TriangleMultiplicationHip
        mod = pm.PairMixerModule()
        assert all(type(layer) is hip_pm.PairMixerLayerHip for layer in mod.layers)
        assert type(mod.msa_layer) is hip_pm.PairMixerMSALayerHip
    assert type(pm.PairMixerModule().layers[0]).__module__ == f"{PKG}.biomoa.modules.pairmixer"


def test_install_unknown_variant_changes_nothing(ref):
    before = _types(ref)
    reg = dict(ref["ops.triangle_multiplication"].REGISTRY)
    with pytest.raises(KeyError, match="bogus"):
        integration.install(PKG, opm_variants=("vanilla", "bogus"))
    assert _types(ref) == before
    assert ref["ops.triangle_multiplication"].REGISTRY == reg


def test_install_missing_package_raises():
    with pytest.raises(ImportError):
        integration.install("no_such_reference_package_here")
