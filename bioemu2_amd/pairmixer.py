"""The reference trunk's PairMixer layers on MI355X, assembled from the HIP ops.

Mirrors ``src/bioemu2/biomoa/modules/pairmixer.py``:

* ``PairMixerLayerHip`` = ``PairMixerLayer`` (:373-456): same constructor
  kwargs, submodules and ``state_dict`` keys (``tri_mul_out``, ``tri_mul_in``,
  ``transition_z``), ``forward(s, z, pair_mask) -> (s, z)`` with
  z += TriMulOut; z += TriMulIn; z += Transition_z.
* ``PairMixerMSALayerHip`` = ``PairMixerMSALayer`` (:614-757): submodules
  ``msa_transition``, ``pair_weighted_averaging``, ``tri_mul_out``,
  ``tri_mul_in``, ``z_transition``, ``outer_product_mean``;
  ``forward(s, z, m, token_mask, msa_mask, chunk_heads_pwa=False) -> (s, z, m)``
  with m += PWA(m, z, token_mask); m += Transition_m(m); z += OPM(m, msa_mask);
  then the three z updates.  ``token_mask`` is the pair mask [B,T,T] (:589).

Inference only: dropout is the identity at eval (biomoa/ops/dropout.py:68-69),
so the dropout rates are accepted and stored.  ``forward_`` updates the
tensors in place: every residual add is fused into the producing kernel and
all ops share one preallocated workspace.  Optional int8 tails carry the
residual streams z and m at ~16 significant bits (pairformer.py explains the
format); ``forward`` always uses them and rounds each stream once.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from .outer_product_mean import REGISTRY as OPM_REGISTRY
from .pair_weighted_averaging import PairWeightedAveraging
from .strategy import make
from .residual import join_stream, split_stream
from .transition import Transition
from .triangle_multiplication import REGISTRY as TRIMUL_REGISTRY


class _WorkspaceMixin:
    _ws: Tensor | None

    def _workspace(self, need: int, device) -> Tensor:
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = _ops.workspace(need, device)
        return self._ws


class PairMixerLayerHip(nn.Module, _WorkspaceMixin):
    def __init__(
        self,
        token_s: int,
        token_z: int,
        dropout: float = 0.25,
        trimul_variant: str = "cueq",
        trimul_tile_size: int | None = None,
        transition_chunk_size: int | None = None,
        trimul_matmul_precision: str | None = None,
    ) -> None:
        super().__init__()
        self.token_z = token_z
        self.dropout = dropout
        self.tri_mul_out = make(TRIMUL_REGISTRY, trimul_variant, dim=token_z, mode="outgoing",
                                tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
        self.tri_mul_in = make(TRIMUL_REGISTRY, trimul_variant, dim=token_z, mode="incoming",
                               tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
        self.transition_z = Transition(dim=token_z, hidden=token_z * 4, chunk_size=transition_chunk_size)
        self._ws = None

    def workspace_bytes(self, B: int, N: int) -> int:
        return max(_ops.trimul_workspace_bytes(B, N, self.token_z),
                   _ops.transition_pair_workspace_bytes(self.token_z, self.transition_z.hidden))

    @torch.no_grad()
    def forward_(
        self, s: Tensor, z: Tensor, pair_mask: Tensor, z_tail: Tensor | None = None
    ) -> tuple[Tensor, Tensor]:
        """In place on bf16 ``z [B,T,T,token_z]`` (and its int8 tail, if given); ``s`` passes through."""
        _ops.require_gpu(z, type(self).__name__)
        B, N = z.shape[0], z.shape[1]
        ws = self._workspace(self.workspace_bytes(B, N), z.device)
        pm = _ops.mask_u8(pair_mask)
        _ops.launch_trimul(z, pm, *self.tri_mul_out.prepared_params(), z, True, residual=True, ws=ws, tail=z_tail)
        _ops.launch_trimul(z, pm, *self.tri_mul_in.prepared_params(), z, False, residual=True, ws=ws, tail=z_tail)
        _ops.launch_transition_pair(z, *self.transition_z.prepared_params(), z, residual=True, ws=ws, tail=z_tail)
        return s, z

    def forward(self, s: Tensor, z: Tensor, pair_mask: Tensor) -> tuple[Tensor, Tensor]:
        z_hi, z_tail = split_stream(z)
        self.forward_(s, z_hi, pair_mask, z_tail)
        return s, join_stream(z_hi, z_tail, z.dtype)


class PairMixerMSALayerHip(nn.Module, _WorkspaceMixin):
    def __init__(
        self,
        token_s: int,
        msa_s: int,
        token_z: int,
        msa_dropout: float,
        z_dropout: float,
        trimul_variant: str = "cueq",
        trimul_tile_size: int | None = None,
        transition_chunk_size: int | None = None,
        opm_variant: str = "vanilla",
        opm_tile_size: int | None = None,
        opm_matmul_precision: str | None = None,
        trimul_matmul_precision: str | None = None,
    ) -> None:
        super().__init__()
        self.msa_s, self.token_z = msa_s, token_z
        self.msa_dropout = msa_dropout
        self.z_dropout = z_dropout
        self.msa_transition = Transition(dim=msa_s, hidden=msa_s * 4, chunk_size=transition_chunk_size)
        self.pair_weighted_averaging = PairWeightedAveraging(c_m=msa_s, c_z=token_z, c_h=32, num_heads=8)
        self.tri_mul_out = make(TRIMUL_REGISTRY, trimul_variant, mode="outgoing", dim=token_z,
                                tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
        self.tri_mul_in = make(TRIMUL_REGISTRY, trimul_variant, mode="incoming", dim=token_z,
                               tile_size=trimul_tile_size, matmul_precision=trimul_matmul_precision)
        self.z_transition = Transition(dim=token_z, hidden=token_z * 4, chunk_size=transition_chunk_size)
        self.outer_product_mean = make(OPM_REGISTRY, opm_variant, c_in=msa_s, c_hidden=32, c_out=token_z,
                                       tile_size=opm_tile_size, matmul_precision=opm_matmul_precision)
        self._ws = None

    def workspace_bytes(self, B: int, S: int, N: int) -> int:
        return max(
            _ops.pwa_workspace_bytes(B, S, N, self.msa_s, 32, 8),
            _ops.transition_pair_workspace_bytes(self.msa_s, self.msa_transition.hidden),
            _ops.opm_workspace_bytes(B, S, N, self.msa_s, 32),
            _ops.trimul_workspace_bytes(B, N, self.token_z),
            _ops.transition_pair_workspace_bytes(self.token_z, self.z_transition.hidden),
        )

    @torch.no_grad()
    def forward_(
        self,
        s: Tensor,
        z: Tensor,
        m: Tensor,
        token_mask: Tensor,
        msa_mask: Tensor,
        chunk_heads_pwa: bool = False,
        z_tail: Tensor | None = None,
        m_tail: Tensor | None = None,
    ) -> tuple[Tensor, Tensor, Tensor]:
        """In place on bf16 ``z [B,T,T,token_z]`` and ``m [B,S,T,msa_s]`` (and their int8 tails, if given);
        ``s`` passes through."""
        _ops.require_gpu(z, type(self).__name__)
        B, S, N = m.shape[0], m.shape[1], m.shape[2]
        ws = self._workspace(self.workspace_bytes(B, S, N), z.device)
        pm = _ops.mask_u8(token_mask)
        _ops.launch_pwa(m, z, pm, *self.pair_weighted_averaging.prepared_params(), m, 8, residual=True, ws=ws,
                        tail=m_tail)
        _ops.launch_transition_pair(m, *self.msa_transition.prepared_params(), m, residual=True, ws=ws, tail=m_tail)
        mask3, mean_rows = _ops.opm_mask3(msa_mask, B, S, N)
        _ops.launch_opm(m, mask3, mean_rows, *self.outer_product_mean.prepared_params(), out=z, z_res=z, ws=ws,
                        tail=z_tail)
        _ops.launch_trimul(z, pm, *self.tri_mul_out.prepared_params(), z, True, residual=True, ws=ws, tail=z_tail)
        _ops.launch_trimul(z, pm, *self.tri_mul_in.prepared_params(), z, False, residual=True, ws=ws, tail=z_tail)
        _ops.launch_transition_pair(z, *self.z_transition.prepared_params(), z, residual=True, ws=ws, tail=z_tail)
        return s, z, m

    def forward(
        self, s: Tensor, z: Tensor, m: Tensor, token_mask: Tensor, msa_mask: Tensor, chunk_heads_pwa: bool = False
    ) -> tuple[Tensor, Tensor, Tensor]:
        (z_hi, z_tail), (m_hi, m_tail) = split_stream(z), split_stream(m)
        self.forward_(s, z_hi, m_hi, token_mask, msa_mask, chunk_heads_pwa, z_tail, m_tail)
        return s, join_stream(z_hi, z_tail, z.dtype), join_stream(m_hi, m_tail, m.dtype)
