"""Variant factory with the reference's ``make()`` contract.

Same behaviour as ``src/bioemu2/biomoa/utils/strategy.py:13-50``: look the
variant up by enum or value, support 2-tuple ``(module, class)`` and 3-tuple
``(module, starting_class, ending_class)`` entries (the latter selected by a
``starting`` kwarg, default True), forward ``matmul_precision`` only when the
class ``__init__`` accepts it, and raise ``ValueError("Unknown variant…")``.
"""

from __future__ import annotations

import importlib
import inspect

import torch.nn as nn


def make(registry: dict, variant: str, *, matmul_precision: str | None = None, **kwargs) -> nn.Module:
    for key in registry:
        if (key == variant) or (getattr(key, "value", None) == variant):
            entry = registry[key]
            if len(entry) == 3:
                mod_path, starting_cls, ending_cls = entry
                starting = kwargs.pop("starting", True)
                cls_name = starting_cls if starting else ending_cls
            else:
                mod_path, cls_name = entry
            cls = getattr(importlib.import_module(mod_path), cls_name)
            if matmul_precision is not None and "matmul_precision" in inspect.signature(cls).parameters:
                kwargs["matmul_precision"] = matmul_precision
            return cls(**kwargs)
    available = [getattr(k, "value", k) for k in registry]
    raise ValueError(f"Unknown variant: {variant!r}, available: {available}")
