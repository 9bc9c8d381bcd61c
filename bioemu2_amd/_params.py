"""Device-ready copies of module parameters, cached until a parameter changes."""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor


class PreparedParams:
    """Caches ``(param.detach().to(dtype).contiguous(), ...)`` for a module.

    The cache key is (data_ptr, version counter, device, dtype) of every
    source parameter, so in-place updates (optimizer steps, ``load_state_dict``)
    and ``.to()`` moves invalidate it.
    """

    def __init__(self, spec: list[tuple[str, torch.dtype]]):
        self.spec = spec
        self._key: tuple | None = None
        self._val: tuple[Tensor, ...] | None = None

    def get(self, module: nn.Module) -> tuple[Tensor, ...]:
        params = [module.get_parameter(name) for name, _ in self.spec]
        key = tuple((p.data_ptr(), p._version, p.device, p.dtype) for p in params)
        if key != self._key or self._val is None:
            self._val = tuple(
                p.detach().to(dtype=dt).contiguous() for p, (_, dt) in zip(params, self.spec)
            )
            self._key = key
        return self._val
