"""Bind the HIP classes into an imported reference package.

The reference builds its hot-path ops in two ways:

* through registries that ``make()`` resolves by variant name
  (utils/strategy.py:13-50): ``REGISTRY`` in ops/triangle_multiplication.py:348-352
  (imported by modules/pairmixer.py:15 as ``TRIMUL_REGISTRY``) and ``REGISTRY`` in
  ops/outer_product_mean.py:155-158 (modules/pairmixer.py:11, ``OPM_REGISTRY``);
* by calling a class that the calling module bound at its own import with
  ``from bioemu2.biomoa.ops.X import Y``: modules/transformer.py:22-23,
  modules/pairmixer.py:13-14, modules/diffusion.py:26 and models/score_model.py:14.
  PairwiseConditioning is defined and used inside modules/diffusion.py (:151, :464).

Rebinding a class in its defining ops module alone misses the second kind, because each
caller holds its own name for it. ``install()`` rebinds the name in every module that binds
it, and points the registry entries (the dicts are shared, so one update reaches every
importer) at the HIP classes. Modules built afterwards construct the HIP classes with the
reference's own kwargs; parameter names and shapes are the reference's, so checkpoints load
unchanged.

Left alone on purpose:

* the ``full`` TriMul variant (the reference's eager PyTorch path, kept for comparison)
  unless ``trimul_variants`` names it;
* ``bioemu2.context_parallel`` (its DTensorAwareTransition subclasses the reference
  Transition at class definition, and sharding across GPUs is outside this library);
* TrunkEmbeddings: the file format is the same both ways, nothing to swap.
"""

from __future__ import annotations

import importlib
from dataclasses import dataclass, field
from typing import Any, Iterable

# (module under the reference package, name bound there, HIP module, HIP class)
CLASS_BINDINGS: tuple[tuple[str, str, str, str], ...] = (
    # definitions (ops/attention_pair_bias.py, ops/transition.py, ops/pair_weighted_averaging.py)
    ("biomoa.ops.attention_pair_bias", "AttentionPairBias", "bioemu2_amd.attention_pair_bias", "AttentionPairBias"),
    ("biomoa.ops.attention_pair_bias", "AttentionPairBiasSlidingWindow", "bioemu2_amd.attention_pair_bias",
     "AttentionPairBiasSlidingWindow"),
    ("biomoa.ops.transition", "Transition", "bioemu2_amd.transition", "Transition"),
    ("biomoa.ops.pair_weighted_averaging", "PairWeightedAveraging", "bioemu2_amd.pair_weighted_averaging",
     "PairWeightedAveraging"),
    ("biomoa.modules.embedders", "DistogramModule", "bioemu2_amd.glue", "DistogramModule"),
    # import-time bindings of the callers
    ("biomoa.modules.transformer", "AttentionPairBias", "bioemu2_amd.attention_pair_bias", "AttentionPairBias"),
    ("biomoa.modules.transformer", "AttentionPairBiasSlidingWindow", "bioemu2_amd.attention_pair_bias",
     "AttentionPairBiasSlidingWindow"),
    ("biomoa.modules.transformer", "Transition", "bioemu2_amd.transition", "Transition"),
    ("biomoa.modules.pairmixer", "Transition", "bioemu2_amd.transition", "Transition"),
    ("biomoa.modules.pairmixer", "PairWeightedAveraging", "bioemu2_amd.pair_weighted_averaging",
     "PairWeightedAveraging"),
    ("biomoa.modules.diffusion", "Transition", "bioemu2_amd.transition", "Transition"),
    ("biomoa.modules.diffusion", "PairwiseConditioning", "bioemu2_amd.glue", "PairwiseConditioning"),
    ("biomoa.models.score_model", "DistogramModule", "bioemu2_amd.glue", "DistogramModule"),
)

# Whole-layer swap (pairmixer.py:373-423, :614-709): PairMixerModule builds its layers inside
# modules/pairmixer.py, so rebinding the names there is enough.
LAYER_BINDINGS: tuple[tuple[str, str, str, str], ...] = (
    ("biomoa.modules.pairmixer", "PairMixerLayer", "bioemu2_amd.pairmixer", "PairMixerLayerHip"),
    ("biomoa.modules.pairmixer", "PairMixerMSALayer", "bioemu2_amd.pairmixer", "PairMixerMSALayerHip"),
)

# (ops module, registry name, HIP (module, class))
REGISTRY_BINDINGS: tuple[tuple[str, str, tuple[str, str]], ...] = (
    ("biomoa.ops.triangle_multiplication", "REGISTRY",
     ("bioemu2_amd.triangle_multiplication", "TriangleMultiplicationHip")),
    ("biomoa.ops.outer_product_mean", "REGISTRY", ("bioemu2_amd.outer_product_mean", "OuterProductMeanHip")),
)

DEFAULT_TRIMUL_VARIANTS = ("cueq", "cueq_tiled")
DEFAULT_OPM_VARIANTS = ("vanilla", "triton_memory_saving")

_MISSING = object()


@dataclass
class Installation:
    """What ``install()`` changed, with the previous values so that ``undo()`` restores them."""

    attributes: list[tuple[Any, str, Any]] = field(default_factory=list)
    registry_entries: list[tuple[dict, Any, Any]] = field(default_factory=list)

    @property
    def bound(self) -> list[str]:
        return [f"{m.__name__}.{name}" for m, name, _ in self.attributes]

    def undo(self) -> None:
        for module, name, old in reversed(self.attributes):
            if old is _MISSING:
                delattr(module, name)
            else:
                setattr(module, name, old)
        for registry, key, old in reversed(self.registry_entries):
            if old is _MISSING:
                del registry[key]
            else:
                registry[key] = old
        self.attributes.clear()
        self.registry_entries.clear()

    def __enter__(self) -> "Installation":
        return self

    def __exit__(self, *exc) -> None:
        self.undo()


def _registry_key(registry: dict, variant: str):
    """The registry key whose value (the enum's ``.value``) or self equals ``variant``, as ``make()`` matches
    them (strategy.py:26-31)."""
    for key in registry:
        if key == variant or getattr(key, "value", _MISSING) == variant:
            return key
    raise KeyError(f"variant {variant!r} not in registry; available: {[getattr(k, 'value', k) for k in registry]}")


def install(
    package: str = "bioemu2",
    *,
    trimul_variants: Iterable[str] = DEFAULT_TRIMUL_VARIANTS,
    opm_variants: Iterable[str] = DEFAULT_OPM_VARIANTS,
    whole_layers: bool = False,
) -> Installation:
    """Rebind the reference's hot-path classes and registry entries to the HIP implementations.

    ``package`` is the reference's top-level package name. Every module named in the binding tables is
    imported (an ImportError names the module). ``whole_layers`` also swaps PairMixerLayer and
    PairMixerMSALayer for the fused HIP layers. Call before the model is built; returns an
    ``Installation`` whose ``undo()`` (or ``with`` exit) restores the previous bindings.
    """
    inst = Installation()
    bindings = CLASS_BINDINGS + (LAYER_BINDINGS if whole_layers else ())
    try:
        for ref_mod, name, hip_mod, hip_name in bindings:
            module = importlib.import_module(f"{package}.{ref_mod}")
            new = getattr(importlib.import_module(hip_mod), hip_name)
            inst.attributes.append((module, name, getattr(module, name, _MISSING)))
            setattr(module, name, new)
        variants = {REGISTRY_BINDINGS[0][0]: tuple(trimul_variants), REGISTRY_BINDINGS[1][0]: tuple(opm_variants)}
        for ref_mod, reg_name, target in REGISTRY_BINDINGS:
            registry = getattr(importlib.import_module(f"{package}.{ref_mod}"), reg_name)
            for variant in variants[ref_mod]:
                key = _registry_key(registry, variant)
                inst.registry_entries.append((registry, key, registry.get(key, _MISSING)))
                registry[key] = target
    except BaseException:
        inst.undo()
        raise
    return inst
