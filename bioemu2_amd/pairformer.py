"""One Pairformer block on MI355X, assembled from the HIP ops.

The reference trunk is a PairMixer stack (``src/bioemu2/biomoa/modules/
pairmixer.py:373-456``: TriMulOut, TriMulIn, Transition on z).  The block
here is the AlphaFold3 Pairformer ordering (suppl. Alg. 17) built from the
reference ops plus triangle attention:

    z += TriMulOut(z, pm); z += TriMulIn(z, pm)
    z += TriAttStart(z, pm); z += TriAttEnd(z, pm); z += Transition_z(z)
    s += AttentionPairBias(s, z, mask)  (initial_norm=True); s += Transition_s(s)

with ``pm = mask_i & mask_j`` (pairmixer.py:263-264) and the residual form of
``PairMixerLayer.forward`` (pairmixer.py:446-456; dropout is the identity at
inference, biomoa/ops/dropout.py:58-70).  ``forward_`` updates ``s`` and ``z``
in place: every residual add is fused into the producing kernel and all ops
share one preallocated workspace, so a block allocates nothing after the
first call at a given shape.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from .attention_pair_bias import AttentionPairBias
from .transition import Transition
from .triangle_attention import TriangleAttentionHip
from .triangle_multiplication import TriangleMultiplicationHip


class PairformerBlockHip(nn.Module):
    def __init__(
        self,
        c_s: int = 384,
        c_z: int = 128,
        triatt_heads: int = 4,
        apb_heads: int = 16,
        transition_factor: int = 4,
    ) -> None:
        super().__init__()
        self.c_s, self.c_z = c_s, c_z
        self.apb_heads = apb_heads
        self.tri_mul_out = TriangleMultiplicationHip(c_z, "outgoing")
        self.tri_mul_in = TriangleMultiplicationHip(c_z, "incoming")
        self.tri_att_start = TriangleAttentionHip(c_z, triatt_heads, starting=True)
        self.tri_att_end = TriangleAttentionHip(c_z, triatt_heads, starting=False)
        self.transition_z = Transition(c_z, transition_factor * c_z)
        self.attention_pair_bias = AttentionPairBias(c_s, c_z, apb_heads, initial_norm=True)
        self.transition_s = Transition(c_s, transition_factor * c_s)
        self._ws: Tensor | None = None
        self._mask_key: tuple | None = None
        self._masks: tuple[Tensor, Tensor] | None = None

    def workspace_bytes(self, B: int, N: int) -> int:
        return max(
            _ops.trimul_workspace_bytes(B, N, self.c_z),
            _ops.triatt_workspace_bytes(B, N, self.c_z, self.tri_att_start.num_heads),
            _ops.apb_workspace_bytes(B, 1, N, self.c_s, self.apb_heads),
            _ops.transition_token_workspace_bytes(B * N, self.c_s, self.transition_s.hidden),
            _ops.transition_pair_workspace_bytes(self.c_z, self.transition_z.hidden),
        )

    def _workspace(self, B: int, N: int, device) -> Tensor:
        need = self.workspace_bytes(B, N)
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = _ops.workspace(need, device)
        return self._ws

    def _pair_masks(self, token_mask: Tensor) -> tuple[Tensor, Tensor]:
        """(token mask, pair mask = mask_i & mask_j) as uint8, cached per mask tensor version."""
        key = (token_mask.data_ptr(), token_mask._version, tuple(token_mask.shape), token_mask.device)
        if key != self._mask_key or self._masks is None:
            m = token_mask.bool()
            self._masks = (_ops.mask_u8(m), _ops.mask_u8(m[:, :, None] & m[:, None, :]))
            self._mask_key = key
        return self._masks

    @torch.no_grad()
    def forward_(self, s: Tensor, z: Tensor, token_mask: Tensor) -> tuple[Tensor, Tensor]:
        """In-place block on bf16 ``s [B,N,c_s]``, ``z [B,N,N,c_z]``, ``token_mask [B,N]``."""
        _ops.require_gpu(z, type(self).__name__)
        B, N = token_mask.shape
        ws = self._workspace(B, N, z.device)
        tok, pm = self._pair_masks(token_mask)
        _ops.launch_trimul(z, pm, *self.tri_mul_out.prepared_params(), z, True, residual=True, ws=ws)
        _ops.launch_trimul(z, pm, *self.tri_mul_in.prepared_params(), z, False, residual=True, ws=ws)
        _ops.launch_triatt(z, pm, *self.tri_att_start.prepared_params(), z, True, residual=True, ws=ws)
        _ops.launch_triatt(z, pm, *self.tri_att_end.prepared_params(), z, False, residual=True, ws=ws)
        _ops.launch_transition_pair(z, *self.transition_z.prepared_params(), z, residual=True, ws=ws)
        _ops.launch_apb(s, z, tok, *self.attention_pair_bias.prepared_params(), s, self.apb_heads,
                        residual=True, ws=ws)
        _ops.launch_transition_token(s, *self.transition_s.prepared_params(), s, residual=True, ws=ws)
        return s, z

    def forward(self, s: Tensor, z: Tensor, token_mask: Tensor) -> tuple[Tensor, Tensor]:
        """Out-of-place block: returns new ``(s, z)`` in the input dtypes."""
        s2 = s.to(torch.bfloat16).contiguous().clone()
        z2 = z.to(torch.bfloat16).contiguous().clone()
        self.forward_(s2, z2, token_mask)
        return s2.to(s.dtype), z2.to(z.dtype)
