"""Pair-tensor glue either side of the trunk on MI355X.

* ``DistogramModule`` mirrors ``src/bioemu2/biomoa/modules/embedders.py:174-206``:
  constructor ``(token_z, num_bins)``, parameter ``distogram`` (``nn.Linear``
  with bias), ``forward(z) = distogram(z + z^T)``.  One HIP kernel computes each
  unordered pair once and writes both (i, j) and (j, i) (the output is exactly
  symmetric).
* ``PairwiseConditioning`` mirrors ``biomoa/modules/diffusion.py:464-535``:
  constructor ``(token_z, dim_token_rel_pos_feats, a_z=None, num_transitions=2,
  transition_expansion_factor=2, transition_chunk_size=None)``, parameters
  ``dim_pairwise_init_proj.{0,1}`` (LayerNorm over the concatenation,
  LinearNoBias) and ``transitions.{k}``; ``forward(z_trunk, token_rel_pos_feats)``.
  The LN + projection is one HIP kernel that reads both inputs in place (no
  concatenated copy); each transition is the fused row kernel with its residual
  add fused, in place.  fp32 inputs with autocast off (the reference runs its
  denoiser so, score_model.py:355) take the fp32 path: fp32 LN over the
  concatenation read in place, fp32 MFMA projection, fp32 transitions with the
  residual fused; any token_z + c_rel multiple of 8 and a_z multiple of 32.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from ._params import PreparedParams
from .residual import join_stream
from .transition import Transition

BF16 = torch.bfloat16


class DistogramModule(nn.Module):
    def __init__(self, token_z: int, num_bins: int) -> None:
        super().__init__()
        self.distogram = nn.Linear(token_z, num_bins)
        self._prepared = PreparedParams([("distogram.weight", BF16), ("distogram.bias", torch.float32)])
        self._prepared32 = PreparedParams([("distogram.weight", torch.float32), ("distogram.bias", torch.float32)])

    def prepared_params(self) -> tuple[Tensor, Tensor]:
        return self._prepared.get(self)

    @torch.no_grad()
    def forward(self, z: Tensor) -> Tensor:
        """bf16 z (or fp32 under bf16 autocast): the bf16 kernel, fp32 accumulation, output in z's dtype; fp32 z
        with autocast off: IEEE fp32 arithmetic."""
        _ops.require_gpu(z, type(self).__name__)
        if _ops.fp32_mode(z):
            w, b = self._prepared32.get(self)
            out = torch.empty(*z.shape[:-1], w.shape[0], dtype=torch.float32, device=z.device)
            return _ops.launch_distogram_f32(z.contiguous(), w, b, out)
        zb = z.to(BF16).contiguous()
        w, b = self.prepared_params()
        # fp32 callers get the fp32 accumulator (no output rounding); others a bf16 output
        odt = torch.float32 if z.dtype == torch.float32 else BF16
        out = torch.empty(*zb.shape[:-1], w.shape[0], dtype=odt, device=zb.device)
        _ops.launch_distogram(zb, w, b, out)
        return out.to(z.dtype)


class PairwiseConditioning(nn.Module):
    def __init__(
        self,
        token_z: int,
        dim_token_rel_pos_feats: int,
        a_z: int | None = None,
        num_transitions: int = 2,
        transition_expansion_factor: int = 2,
        transition_chunk_size: int | None = None,
    ) -> None:
        super().__init__()
        a_z = a_z if a_z is not None else token_z
        self.a_z = a_z
        self.token_z, self.c_rel = token_z, dim_token_rel_pos_feats
        self.dim_pairwise_init_proj = nn.Sequential(
            nn.LayerNorm(token_z + dim_token_rel_pos_feats),
            nn.Linear(token_z + dim_token_rel_pos_feats, a_z, bias=False),
        )
        self.transitions = nn.ModuleList(
            [
                Transition(dim=a_z, hidden=transition_expansion_factor * a_z, chunk_size=transition_chunk_size)
                for _ in range(num_transitions)
            ]
        )
        self._prepared = PreparedParams([
            ("dim_pairwise_init_proj.0.weight", torch.float32),
            ("dim_pairwise_init_proj.0.bias", torch.float32),
            ("dim_pairwise_init_proj.1.weight", BF16),
        ])
        self._prepared32 = PreparedParams([
            ("dim_pairwise_init_proj.0.weight", torch.float32),
            ("dim_pairwise_init_proj.0.bias", torch.float32),
            ("dim_pairwise_init_proj.1.weight", torch.float32),
        ])
        self._ws: Tensor | None = None

    def prepared_params(self) -> tuple[Tensor, Tensor, Tensor]:
        return self._prepared.get(self)

    def prepared_params_f32(self) -> tuple[Tensor, Tensor, Tensor]:
        return self._prepared32.get(self)

    def _workspace(self, device) -> Tensor:
        t0 = self.transitions[0] if len(self.transitions) else None
        need = _ops.pair_cond_workspace_bytes(self.token_z, self.c_rel, self.a_z)
        if t0 is not None:
            need = max(need, _ops.transition_pair_workspace_bytes(self.a_z, t0.hidden))
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = _ops.workspace(need, device)
        return self._ws

    def _forward_f32(self, z_trunk: Tensor, token_rel_pos_feats: Tensor) -> Tensor:
        z = z_trunk.contiguous()
        rel = token_rel_pos_feats.to(torch.float32).contiguous()
        P = z.numel() // z.shape[-1]
        need = _ops.pair_cond_f32_workspace_bytes(P, self.token_z, self.c_rel)
        for t in self.transitions:
            need = max(need, _ops.transition_f32_workspace_bytes(P, self.a_z, t.hidden))
        ws = _ops.workspace(need, z.device)
        out = torch.empty(*z.shape[:-1], self.a_z, dtype=torch.float32, device=z.device)
        _ops.launch_pair_cond_proj_f32(z, rel, *self.prepared_params_f32(), out, ws=ws)
        for transition in self.transitions:   # z = transition(z) + z, residual fused, in place
            _ops.launch_transition_f32(out, *transition.prepared_params_f32(), out, residual=True, ws=ws)
        return out

    @torch.no_grad()
    def forward(self, z_trunk: Tensor, token_rel_pos_feats: Tensor) -> Tensor:
        _ops.require_gpu(z_trunk, type(self).__name__)
        if _ops.fp32_mode(z_trunk):
            return self._forward_f32(z_trunk, token_rel_pos_feats)
        z = z_trunk.to(BF16).contiguous()
        rel = token_rel_pos_feats.to(BF16).contiguous()
        ws = self._workspace(z.device)
        # the conditioning stream is carried as bf16 + int8 tail through the residual transitions and
        # rounded once at the end (to bf16, or not at all for an fp32 caller under autocast)
        out = torch.empty(*z.shape[:-1], self.a_z, dtype=BF16, device=z.device)
        tail = torch.empty(out.shape, dtype=torch.int8, device=z.device)
        _ops.launch_pair_cond_proj(z, rel, *self.prepared_params(), out, ws=ws, out_tail=tail)
        for transition in self.transitions:   # z = transition(z) + z, fused and in place
            _ops.launch_transition_pair(out, *transition.prepared_params(), out, residual=True, ws=ws, tail=tail)
        return join_stream(out, tail, z_trunk.dtype)
