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
inference, biomoa/ops/dropout.py:58-70).

Residual streams.  ``forward_`` updates bf16 ``s`` and ``z`` in place, with
every residual add fused into the producing kernel.  Given int8 tail planes
(``s_tail``, ``z_tail``; see ``include/bioemu2_mi355x.h``, "Residual tails"),
the streams are carried at ~16 significant bits: each op adds its update to
value + tail and writes back a bf16 value and a new tail, so a stack of ops
rounds once, when the stream is joined, instead of after every add as the
reference's bf16-autocast trunk does (bf16 z + bf16 update under autocast,
pairmixer.py:446-456, model.py:216-223).  ``forward`` always carries tails:
fp32 inputs are split into (bf16, tail) and the result joined back to fp32;
bf16 inputs start with zero tails and the result is rounded once.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _ops
from .attention_pair_bias import AttentionPairBias
from .residual import join_stream, split_stream
from .transition import Transition
from .triangle_attention import TriangleAttentionHip
from .triangle_multiplication import TriangleMultiplicationHip


def pair_masks(token_mask: Tensor) -> tuple[Tensor, Tensor]:
    """(token mask, pair mask = mask_i & mask_j) as uint8 (pairmixer.py:263-264)."""
    m = token_mask.bool()
    return _ops.mask_u8(m), _ops.mask_u8(m[:, :, None] & m[:, None, :])


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

    @torch.no_grad()
    def forward_(
        self,
        s: Tensor,
        z: Tensor,
        token_mask: Tensor,
        s_tail: Tensor | None = None,
        z_tail: Tensor | None = None,
        ws: Tensor | None = None,
        masks: tuple[Tensor, Tensor] | None = None,
    ) -> tuple[Tensor, Tensor]:
        """In-place block on bf16 ``s [B,N,c_s]``, ``z [B,N,N,c_z]``, ``token_mask [B,N]``.

        ``s_tail`` / ``z_tail``: int8 tails of the residual streams (same shapes), updated in place;
        ``None`` keeps that stream in plain bf16.  ``ws``: a caller-owned workspace of at least
        ``workspace_bytes(B, N)`` bytes (default: one the block caches per shape).  ``masks``: the
        ``pair_masks(token_mask)`` pair, built once by a caller that runs many blocks or steps on the
        same mask (default: built from ``token_mask`` here, two small allocations per call).
        """
        _ops.require_gpu(z, type(self).__name__)
        B, N = token_mask.shape
        if ws is None:
            ws = self._workspace(B, N, z.device)
        tok, pm = masks if masks is not None else pair_masks(token_mask)
        _ops.launch_trimul(z, pm, *self.tri_mul_out.prepared_params(), z, True, residual=True, ws=ws, tail=z_tail)
        _ops.launch_trimul(z, pm, *self.tri_mul_in.prepared_params(), z, False, residual=True, ws=ws, tail=z_tail)
        _ops.launch_triatt(z, pm, *self.tri_att_start.prepared_params(), z, True, residual=True, ws=ws, tail=z_tail)
        _ops.launch_triatt(z, pm, *self.tri_att_end.prepared_params(), z, False, residual=True, ws=ws, tail=z_tail)
        _ops.launch_transition_pair(z, *self.transition_z.prepared_params(), z, residual=True, ws=ws, tail=z_tail)
        _ops.launch_apb(s, z, tok, *self.attention_pair_bias.prepared_params(), s, self.apb_heads,
                        residual=True, ws=ws, tail=s_tail)
        _ops.launch_transition_token(s, *self.transition_s.prepared_params(), s, residual=True, ws=ws,
                                     tail=s_tail)
        return s, z

    def workspace_bytes_f32(self, B: int, N: int) -> int:
        return max(
            _ops.trimul_f32_workspace_bytes(B, N, self.c_z),
            _ops.triatt_f32_workspace_bytes(B, N, self.c_z, self.tri_att_start.num_heads),
            _ops.apb_f32_workspace_bytes(B, 1, N, self.c_s, self.apb_heads),
            _ops.transition_f32_workspace_bytes(B * N, self.c_s, self.transition_s.hidden),
            _ops.transition_f32_workspace_bytes(B * N * N, self.c_z, self.transition_z.hidden),
        )

    @torch.no_grad()
    def forward_f32_(self, s: Tensor, z: Tensor, token_mask: Tensor, ws: Tensor | None = None
                     ) -> tuple[Tensor, Tensor]:
        """In place on fp32 ``s [B,N,c_s]`` and ``z [B,N,N,c_z]`` in fp32 arithmetic (fp32 inputs with autocast
        off), in the order of ``forward_``; ``ws``: at least ``workspace_bytes_f32(B, N)`` bytes."""
        _ops.require_gpu(z, type(self).__name__)
        B, N = token_mask.shape
        if ws is None:
            need = self.workspace_bytes_f32(B, N)
            if self._ws is None or self._ws.numel() < need or self._ws.device != z.device:
                self._ws = _ops.workspace(need, z.device)
            ws = self._ws
        tok, pm = pair_masks(token_mask)
        _ops.launch_trimul_f32(z, pm, *self.tri_mul_out.prepared_params_f32(), z, True, residual=True, ws=ws)
        _ops.launch_trimul_f32(z, pm, *self.tri_mul_in.prepared_params_f32(), z, False, residual=True, ws=ws)
        heads = self.tri_att_start.num_heads
        _ops.launch_triatt_f32(z, pm, *self.tri_att_start.prepared_params_f32(), z, True, heads, residual=True, ws=ws)
        _ops.launch_triatt_f32(z, pm, *self.tri_att_end.prepared_params_f32(), z, False, heads, residual=True, ws=ws)
        _ops.launch_transition_f32(z, *self.transition_z.prepared_params_f32(), z, residual=True, ws=ws)
        _ops.launch_apb_f32(s, z, tok, *self.attention_pair_bias.prepared_params_f32(), s, self.apb_heads,
                            residual=True, ws=ws)
        _ops.launch_transition_f32(s, *self.transition_s.prepared_params_f32(), s, residual=True, ws=ws)
        return s, z

    def forward(self, s: Tensor, z: Tensor, token_mask: Tensor) -> tuple[Tensor, Tensor]:
        """Out-of-place block: returns new ``(s, z)`` in the input dtypes.  fp32 inputs with autocast off compute
        in fp32 throughout (``forward_f32_`` on copies); otherwise the bf16 path with the streams carried with
        tails."""
        _ops.require_gpu(z, type(self).__name__)
        if _ops.fp32_mode(z):
            s32, z32 = s.to(torch.float32).contiguous().clone(), z.contiguous().clone()
            return self.forward_f32_(s32, z32, token_mask)
        (s_hi, s_tail), (z_hi, z_tail) = split_stream(s), split_stream(z)
        self.forward_(s_hi, z_hi, token_mask, s_tail, z_tail)
        return join_stream(s_hi, s_tail, s.dtype), join_stream(z_hi, z_tail, z.dtype)

    @torch.no_grad()
    def capture(
        self,
        s: Tensor,
        z: Tensor,
        token_mask: Tensor,
        s_tail: Tensor | None = None,
        z_tail: Tensor | None = None,
    ) -> "BlockGraph":
        """Captures ``forward_`` on these exact buffers into a HIP graph (see ``BlockGraph``)."""
        return BlockGraph(self, s, z, token_mask, s_tail, z_tail)


class BlockGraph:
    """A HIP graph of one in-place ``PairformerBlockHip.forward_`` on fixed buffers.

    The graph owns its workspace and holds references to every tensor its
    kernels read or write: the caller's ``s``, ``z``, tails and token mask, the
    prepared weights of the moment of capture, and the masks built inside the
    capture (graph-pool memory).  Eager calls of the block at other shapes or
    masks therefore cannot free anything a replay touches.  ``replay()``
    re-runs the block on the current contents of those buffers; later weight
    updates are not seen (capture again after changing parameters).
    """

    def __init__(self, block: PairformerBlockHip, s, z, token_mask, s_tail=None, z_tail=None):
        B, N = token_mask.shape
        self.tensors = (s, z, token_mask, s_tail, z_tail)
        self.ws = _ops.workspace(block.workspace_bytes(B, N), z.device)
        # Prepare the weights outside the capture (their conversions allocate and copy).
        mods = (block.tri_mul_out, block.tri_mul_in, block.tri_att_start, block.tri_att_end, block.transition_z,
                block.attention_pair_bias, block.transition_s)
        self.params = tuple(m.prepared_params() for m in mods)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            block.forward_(s, z, token_mask, s_tail, z_tail, ws=self.ws)

    def replay(self) -> None:
        self.graph.replay()
