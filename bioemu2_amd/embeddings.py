"""Trunk embeddings and their on-disk format.

Mirrors ``TrunkEmbeddings`` (``src/bioemu2/biomoa/models/score_model.py:30-78``)
so embeddings produced by the HIP trunk are written in the reference's format
and the reference reads them back unchanged (and vice versa):

* one file per embedding set, written by ``torch.save`` of a plain ``dict``
  mapping exactly the five field names (``s_inputs``, ``single``, ``pair``,
  ``relative_position_encoding``, ``distogram``) to host tensors;
* ``save`` refuses to overwrite an existing file (``FileExistsError``) and
  creates missing parent directories;
* ``load`` uses ``torch.load(..., weights_only=True)`` and rejects anything that
  is not such a dict of tensors (``ValueError``), then moves every tensor to
  ``device``.

Tensors keep their dtype (bf16 from the HIP trunk) and shape.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from pathlib import Path

import torch


@dataclass
class TrunkEmbeddings:
    s_inputs: torch.Tensor
    single: torch.Tensor
    pair: torch.Tensor
    relative_position_encoding: torch.Tensor
    distogram: torch.Tensor

    def save(self, path: Path) -> None:
        path = Path(path)
        if path.exists():
            raise FileExistsError(f"Refusing to overwrite existing file {path}; pass a new path.")
        path.parent.mkdir(parents=True, exist_ok=True)
        torch.save({f.name: getattr(self, f.name).detach().cpu() for f in fields(self)}, path)

    @classmethod
    def load(cls, path: Path, device: torch.device) -> "TrunkEmbeddings":
        tensors = torch.load(Path(path), map_location="cpu", weights_only=True)
        names = {f.name for f in fields(cls)}
        if (
            not isinstance(tensors, dict)
            or set(tensors) != names
            or not all(isinstance(v, torch.Tensor) for v in tensors.values())
        ):
            raise ValueError(f"Invalid trunk embeddings at {path}")
        return cls(**{name: tensors[name].to(device) for name in names})
