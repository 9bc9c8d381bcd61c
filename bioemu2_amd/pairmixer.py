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

    def workspace_bytes_f32(self, B: int, N: int) -> int:
        return max(_ops.trimul_f32_workspace_bytes(B, N, self.token_z),
                   _ops.transition_f32_workspace_bytes(B * N * N, self.token_z, self.transition_z.hidden))

    @torch.no_grad()
    def forward_(
        self, s: Tensor, z: Tensor, pair_mask: Tensor, z_tail: Tensor | None = None, ws: Tensor | None = None
    ) -> tuple[Tensor, Tensor]:
        """In place on bf16 ``z [B,T,T,token_z]`` (and its int8 tail, if given); ``s`` passes through.
        ``ws``: a caller-owned workspace of ``workspace_bytes`` (default: one cached per layer)."""
        _ops.require_gpu(z, type(self).__name__)
        B, N = z.shape[0], z.shape[1]
        if ws is None:
            ws = self._workspace(self.workspace_bytes(B, N), z.device)
        pm = _ops.mask_u8(pair_mask)
        _ops.launch_trimul(z, pm, *self.tri_mul_out.prepared_params(), z, True, residual=True, ws=ws, tail=z_tail)
        _ops.launch_trimul(z, pm, *self.tri_mul_in.prepared_params(), z, False, residual=True, ws=ws, tail=z_tail)
        _ops.launch_transition_pair(z, *self.transition_z.prepared_params(), z, residual=True, ws=ws, tail=z_tail)
        return s, z

    @torch.no_grad()
    def forward_f32_(self, s: Tensor, z: Tensor, pair_mask: Tensor, ws: Tensor | None = None
                     ) -> tuple[Tensor, Tensor]:
        """In place on fp32 ``z`` in IEEE fp32 arithmetic (the reference run with autocast off): the two
        triangle multiplications and the transition, each adding its update into z."""
        _ops.require_gpu(z, type(self).__name__)
        if ws is None:
            ws = self._workspace(self.workspace_bytes_f32(z.shape[0], z.shape[1]), z.device)
        pm = _ops.mask_u8(pair_mask)
        _ops.launch_trimul_f32(z, pm, *self.tri_mul_out.prepared_params_f32(), z, True, residual=True, ws=ws)
        _ops.launch_trimul_f32(z, pm, *self.tri_mul_in.prepared_params_f32(), z, False, residual=True, ws=ws)
        _ops.launch_transition_f32(z, *self.transition_z.prepared_params_f32(), z, residual=True, ws=ws)
        return s, z

    def forward(self, s: Tensor, z: Tensor, pair_mask: Tensor) -> tuple[Tensor, Tensor]:
        """bf16 (or fp32 under bf16 autocast): the bf16 path with z carried as bf16 + int8 tail; fp32 with
        autocast off: IEEE fp32 arithmetic."""
        _ops.require_gpu(z, type(self).__name__)
        if _ops.fp32_mode(z):
            z32 = z.contiguous().clone()
            self.forward_f32_(s, z32, pair_mask)
            return s, z32
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

    def workspace_bytes_f32(self, B: int, S: int, N: int) -> int:
        return max(
            _ops.pwa_f32_workspace_bytes(B, S, N, self.msa_s, 32, 8),
            _ops.transition_f32_workspace_bytes(B * S * N, self.msa_s, self.msa_transition.hidden),
            _ops.opm_f32_workspace_bytes(B, S, N, self.msa_s, 32),
            _ops.trimul_f32_workspace_bytes(B, N, self.token_z),
            _ops.transition_f32_workspace_bytes(B * N * N, self.token_z, self.z_transition.hidden),
        )

    @torch.no_grad()
    def forward_f32_(self, s: Tensor, z: Tensor, m: Tensor, token_mask: Tensor, msa_mask: Tensor,
                     ws: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
        """In place on fp32 ``z`` and ``m`` in IEEE fp32 arithmetic (the reference run with autocast off),
        in the order of ``forward_``: pair-weighted averaging and the MSA transition into m, the outer-product
        mean into z, then the two triangle multiplications and the pair transition."""
        _ops.require_gpu(z, type(self).__name__)
        B, S, N = m.shape[0], m.shape[1], m.shape[2]
        if ws is None:
            ws = self._workspace(self.workspace_bytes_f32(B, S, N), z.device)
        pm = _ops.mask_u8(token_mask)
        pwa = self.pair_weighted_averaging
        _ops.launch_pwa_f32(m, z, pm, *pwa.prepared_params_f32(), m, pwa.num_heads, residual=True, inf=pwa.inf,
                            ws=ws)
        _ops.launch_transition_f32(m, *self.msa_transition.prepared_params_f32(), m, residual=True, ws=ws)
        mask3, mean_rows = _ops.opm_mask3(msa_mask, B, S, N)
        _ops.launch_opm_f32(m, mask3, mean_rows, *self.outer_product_mean.prepared_params_f32(), out=z, z_res=z, ws=ws)
        _ops.launch_trimul_f32(z, pm, *self.tri_mul_out.prepared_params_f32(), z, True, residual=True, ws=ws)
        _ops.launch_trimul_f32(z, pm, *self.tri_mul_in.prepared_params_f32(), z, False, residual=True, ws=ws)
        _ops.launch_transition_f32(z, *self.z_transition.prepared_params_f32(), z, residual=True, ws=ws)
        return s, z, m

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
        ws: Tensor | None = None,
    ) -> tuple[Tensor, Tensor, Tensor]:
        """In place on bf16 ``z [B,T,T,token_z]`` and ``m [B,S,T,msa_s]`` (and their int8 tails, if given);
        ``s`` passes through.  ``ws``: a caller-owned workspace of ``workspace_bytes`` (default: cached)."""
        _ops.require_gpu(z, type(self).__name__)
        B, S, N = m.shape[0], m.shape[1], m.shape[2]
        if ws is None:
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
        """bf16 (or fp32 under bf16 autocast): z and m carried as bf16 + int8 tails; fp32 with autocast off:
        IEEE fp32 arithmetic on fp32 copies of z and m."""
        _ops.require_gpu(z, type(self).__name__)
        if _ops.fp32_mode(z):
            z32, m32 = z.contiguous().clone(), m.to(torch.float32).contiguous().clone()
            self.forward_f32_(s, z32, m32, token_mask, msa_mask)
            return s, z32, m32
        (z_hi, z_tail), (m_hi, m_tail) = split_stream(z), split_stream(m)
        self.forward_(s, z_hi, m_hi, token_mask, msa_mask, chunk_heads_pwa, z_tail, m_tail)
        return s, join_stream(z_hi, z_tail, z.dtype), join_stream(m_hi, m_tail, m.dtype)


NUM_TOKENS = 33   # len(Token) of the reference's token vocabulary (data_interface/const.py:23-57)


class PairMixerModuleHip(nn.Module, _WorkspaceMixin):
    """``PairMixerModule`` (pairmixer.py:299-370): ``num_blocks`` PairMixer layers in order, with the same
    constructor kwargs and ``layers.{i}.*`` keys.  ``forward_`` runs them in place on one z stream (and its
    tail) with one workspace shared by every layer."""

    def __init__(
        self,
        token_s: int,
        token_z: int,
        num_blocks: int,
        dropout: float = 0.25,
        trimul_variant: str = "cueq",
        trimul_tile_size: int | None = None,
        transition_chunk_size: int | None = None,
        trimul_matmul_precision: str | None = None,
    ) -> None:
        super().__init__()
        self.token_z = token_z
        self.num_blocks = num_blocks
        self.dropout = dropout
        self.layers = nn.ModuleList([
            PairMixerLayerHip(token_s, token_z, dropout, trimul_variant=trimul_variant,
                              trimul_tile_size=trimul_tile_size, transition_chunk_size=transition_chunk_size,
                              trimul_matmul_precision=trimul_matmul_precision)
            for _ in range(num_blocks)
        ])
        self._ws = None

    def workspace_bytes(self, B: int, N: int) -> int:
        return self.layers[0].workspace_bytes(B, N) if len(self.layers) else 16

    @torch.no_grad()
    def forward_(self, s: Tensor, z: Tensor, pair_mask: Tensor, z_tail: Tensor | None = None,
                 ws: Tensor | None = None) -> tuple[Tensor, Tensor]:
        _ops.require_gpu(z, type(self).__name__)
        if ws is None:
            ws = self._workspace(self.workspace_bytes(z.shape[0], z.shape[1]), z.device)
        pm = pair_mask.bool()
        for layer in self.layers:   # pairmixer.py:368-369
            layer.forward_(s, z, pm, z_tail, ws=ws)
        return s, z

    def forward(self, s: Tensor, z: Tensor, pair_mask: Tensor) -> tuple[Tensor, Tensor]:
        """bf16 (or fp32 under bf16 autocast): one bf16 + int8-tail z stream through every layer; fp32 with
        autocast off: every layer in IEEE fp32 arithmetic on one fp32 z."""
        _ops.require_gpu(z, type(self).__name__)
        if _ops.fp32_mode(z):
            z32 = z.contiguous().clone()
            ws = self._workspace(self.layers[0].workspace_bytes_f32(z.shape[0], z.shape[1]), z.device) \
                if len(self.layers) else None
            for layer in self.layers:   # pairmixer.py:368-369
                layer.forward_f32_(s, z32, pair_mask, ws=ws)
            return s, z32
        z_hi, z_tail = split_stream(z)
        self.forward_(s, z_hi, pair_mask, z_tail)
        return s, join_stream(z_hi, z_tail, z.dtype)


class PairMixerMSAModuleHip(nn.Module, _WorkspaceMixin):
    """``PairMixerMSAModule`` (pairmixer.py:459-611): same constructor kwargs and keys (``s_proj``,
    ``msa_proj``, ``layers.{i}.*``).  The input embedding m = msa_proj(cat(msa, has_deletion,
    deletion_value[, msa_paired])) + s_proj(emb) is one fp32 HIP kernel writing the MSA stream (bf16 + tail);
    the MSA layers then update z and m in place.  The projection weights are kept in fp32 like the reference's
    parameters; the feature tensors are taken as fp32."""

    def __init__(
        self,
        token_s: int,
        msa_s: int,
        token_z: int,
        s_input_dim: int,
        msa_blocks: int,
        msa_dropout: float,
        z_dropout: float,
        use_paired_feature: bool = False,
        trimul_variant: str = "cueq",
        trimul_tile_size: int | None = None,
        transition_chunk_size: int | None = None,
        opm_variant: str = "vanilla",
        opm_tile_size: int | None = None,
        pwa_chunk_heads: bool = False,
        opm_matmul_precision: str | None = None,
        trimul_matmul_precision: str | None = None,
        num_tokens: int = NUM_TOKENS,
    ) -> None:
        super().__init__()
        self.msa_s, self.token_z = msa_s, token_z
        self.msa_blocks = msa_blocks
        self.msa_dropout = msa_dropout
        self.z_dropout = z_dropout
        self.use_paired_feature = use_paired_feature
        self.pwa_chunk_heads = pwa_chunk_heads
        self.s_proj = nn.Linear(s_input_dim, msa_s, bias=False)
        self.msa_proj = nn.Linear(num_tokens + 2 + int(use_paired_feature), msa_s, bias=False)
        self.layers = nn.ModuleList([
            PairMixerMSALayerHip(token_s, msa_s, token_z, msa_dropout, z_dropout, trimul_variant=trimul_variant,
                                 trimul_tile_size=trimul_tile_size, transition_chunk_size=transition_chunk_size,
                                 opm_variant=opm_variant, opm_tile_size=opm_tile_size,
                                 opm_matmul_precision=opm_matmul_precision,
                                 trimul_matmul_precision=trimul_matmul_precision)
            for _ in range(msa_blocks)
        ])
        self._ws = None

    def workspace_bytes(self, B: int, S: int, N: int) -> int:
        layer = self.layers[0].workspace_bytes(B, S, N) if len(self.layers) else 16
        return max(layer, int(_ops.lib().bioemu_msa_embed_workspace_bytes(B, N)))

    def workspace_bytes_f32(self, B: int, S: int, N: int) -> int:
        layer = self.layers[0].workspace_bytes_f32(B, S, N) if len(self.layers) else 16
        return max(layer, int(_ops.lib().bioemu_msa_embed_workspace_bytes(B, N)))

    @torch.no_grad()
    def forward_f32_(self, z: Tensor, emb: Tensor, msa: Tensor, msa_mask: Tensor, has_deletion: Tensor,
                     deletion_value: Tensor, msa_paired: Tensor, token_pad_mask: Tensor,
                     ws: Tensor | None = None) -> Tensor:
        """In place on fp32 ``z`` in IEEE fp32 arithmetic (a trunk run with autocast off): the fp32 MSA stream
        from the features, then every MSA layer's fp32 path."""
        _ops.require_gpu(z, type(self).__name__)
        B, R, T = msa.shape[:3]
        if ws is None:
            ws = self._workspace(self.workspace_bytes_f32(B, R, T), z.device)
        f32 = torch.float32
        m = torch.empty(B, R, T, self.msa_s, dtype=f32, device=msa.device)
        _ops.launch_msa_embed_f32(
            msa.to(f32).contiguous(), has_deletion.to(f32).contiguous(), deletion_value.to(f32).contiguous(),
            msa_paired.to(f32).contiguous() if self.use_paired_feature else None, emb.to(f32).contiguous(),
            self.msa_proj.weight.to(f32).contiguous(), self.s_proj.weight.to(f32).contiguous(), m, ws=ws)
        tok = token_pad_mask.bool()
        pm = tok[:, :, None] & tok[:, None, :]                       # :589
        for layer in self.layers:                                     # :602-610
            layer.forward_f32_(None, z, m, pm, msa_mask, ws=ws)
        return z

    def embed(self, emb: Tensor, msa: Tensor, has_deletion: Tensor, deletion_value: Tensor, msa_paired: Tensor,
              ws: Tensor | None = None) -> tuple[Tensor, Tensor]:
        """The MSA stream (m [B,R,T,msa_s] bf16, its int8 tail) from the features (pairmixer.py:591-599)."""
        B, R, T = msa.shape[:3]
        f32 = torch.float32
        m = torch.empty(B, R, T, self.msa_s, dtype=torch.bfloat16, device=msa.device)
        m_tail = torch.empty(B, R, T, self.msa_s, dtype=torch.int8, device=msa.device)
        _ops.launch_msa_embed(
            msa.to(f32).contiguous(), has_deletion.to(f32).contiguous(), deletion_value.to(f32).contiguous(),
            msa_paired.to(f32).contiguous() if self.use_paired_feature else None, emb.to(f32).contiguous(),
            self.msa_proj.weight.to(f32).contiguous(), self.s_proj.weight.to(f32).contiguous(), m, m_tail, ws=ws)
        return m, m_tail

    @torch.no_grad()
    def forward_(self, z: Tensor, emb: Tensor, msa: Tensor, msa_mask: Tensor, has_deletion: Tensor,
                 deletion_value: Tensor, msa_paired: Tensor, token_pad_mask: Tensor, z_tail: Tensor | None = None,
                 ws: Tensor | None = None) -> Tensor:
        """In place on the bf16 pair stream ``z`` (and its tail); returns z."""
        _ops.require_gpu(z, type(self).__name__)
        B, R, T = msa.shape[:3]
        if ws is None:
            ws = self._workspace(self.workspace_bytes(B, R, T), z.device)
        m, m_tail = self.embed(emb, msa, has_deletion, deletion_value, msa_paired, ws=ws)
        tok = token_pad_mask.bool()
        pm = tok[:, :, None] & tok[:, None, :]                       # :589
        for layer in self.layers:                                     # :602-610
            layer.forward_(None, z, m, pm, msa_mask, False, z_tail, m_tail, ws=ws)
        return z

    def forward(self, s, z, emb, msa, msa_mask, has_deletion, deletion_value, msa_paired, token_pad_mask):
        """bf16 (or fp32 under bf16 autocast): z carried as bf16 + int8 tail; fp32 with autocast off: IEEE fp32
        arithmetic on an fp32 copy of z."""
        _ops.require_gpu(z, type(self).__name__)
        if _ops.fp32_mode(z):
            z32 = z.contiguous().clone()
            self.forward_f32_(z32, emb, msa, msa_mask, has_deletion, deletion_value, msa_paired, token_pad_mask)
            return s, z32
        z_hi, z_tail = split_stream(z)
        self.forward_(z_hi, emb, msa, msa_mask, has_deletion, deletion_value, msa_paired, token_pad_mask, z_tail)
        return s, join_stream(z_hi, z_tail, z.dtype)


class PairMixerTrunkHip(nn.Module, _WorkspaceMixin):
    """The trunk of ``PairMixerSequenceEmbedder`` (pairmixer.py:23-296) from the initial embeddings on.

    Submodules carry the reference's names (``s_recycle``, ``z_recycle``, ``s_norm``, ``z_norm``,
    ``msa_module``, ``pairmixer_module``), so the trunk part of a reference state_dict loads unchanged
    (``strict=False`` skips the embedder's input layers, relative-position encoder and conditioning, which
    stay with the caller).  ``forward(s_init, z_init, s_inputs, feats, num_steps_recycle)`` runs the recycling
    loop of :275-296: s and z start at zero; every pass sets s = s_init + s_recycle(s_norm(s)) and
    z = z_init + z_recycle(z_norm(z)), runs the MSA module (single updates off) and the PairMixer stack.
    z is carried as one bf16 + tail stream through every pass; s and z come back in s_init's / z_init's dtype.
    With ``use_unconditional_branch=True`` the trunk also holds ``uncond_transition`` (:193-200), and
    ``forward(..., unconditional=True)`` returns s_init and z_init + uncond_transition(z_norm(z_init))
    (:266-273) without running the recycling loop.
    """

    def __init__(
        self,
        token_s: int,
        token_z: int,
        s_input_dim: int,
        msa_s: int = 64,
        msa_blocks: int = 4,
        msa_dropout: float = 0.15,
        z_dropout: float = 0.25,
        num_blocks: int = 48,
        dropout: float = 0.0,
        trimul_variant: str = "cueq",
        opm_variant: str = "vanilla",
        use_paired_feature: bool = True,
        num_tokens: int = NUM_TOKENS,
        use_unconditional_branch: bool = False,
        transition_chunk_size: int | None = None,
    ) -> None:
        super().__init__()
        self.msa_module = PairMixerMSAModuleHip(token_s, msa_s, token_z, s_input_dim, msa_blocks, msa_dropout,
                                                z_dropout, use_paired_feature=use_paired_feature,
                                                trimul_variant=trimul_variant, opm_variant=opm_variant,
                                                num_tokens=num_tokens)
        self.pairmixer_module = PairMixerModuleHip(token_s, token_z, num_blocks, dropout,
                                                   trimul_variant=trimul_variant)
        self.s_recycle = nn.Linear(token_s, token_s, bias=False)     # :186-191
        self.z_recycle = nn.Linear(token_z, token_z, bias=False)
        self.s_norm = nn.LayerNorm(token_s)
        self.z_norm = nn.LayerNorm(token_z)
        # Unconditional branch (:193-200): z = z_init + uncond_transition(z_norm(z_init)).
        self.use_unconditional_branch = use_unconditional_branch
        if use_unconditional_branch:
            self.uncond_transition = Transition(dim=token_z, hidden=token_z * 4, chunk_size=transition_chunk_size)
        self._ws = None

    def workspace_bytes(self, B: int, S: int, N: int, token_s: int) -> int:
        return max(self.msa_module.workspace_bytes(B, S, N), self.pairmixer_module.workspace_bytes(B, N),
                   int(_ops.lib().bioemu_pair_ln_linear_workspace_bytes(self.z_recycle.in_features)),
                   int(_ops.lib().bioemu_token_ln_linear_workspace_bytes(B * N, token_s)))

    def workspace_bytes_f32(self, B: int, S: int, N: int, token_s: int) -> int:
        return max(self.msa_module.workspace_bytes_f32(B, S, N),
                   self.pairmixer_module.layers[0].workspace_bytes_f32(B, N) if len(self.pairmixer_module.layers)
                   else 16,
                   int(_ops.lib().bioemu_ln_linear_f32_workspace_bytes(B * N * N, self.z_recycle.in_features)),
                   int(_ops.lib().bioemu_ln_linear_f32_workspace_bytes(B * N, token_s)))

    @torch.no_grad()
    def forward_unconditional(self, s_init: Tensor, z_init: Tensor) -> tuple[Tensor, Tensor]:
        """The unconditional branch (pairmixer.py:266-273): s = s_init and z = z_init + uncond_transition(
        z_norm(z_init)), one HIP entry (LayerNorm, fused row transition with z_init as the residual base)."""
        if not self.use_unconditional_branch:
            raise ValueError(
                "Passing unconditional=True at inference time requires use_unconditional_branch=True at __init__"
            )
        _ops.require_gpu(z_init, type(self).__name__)
        D = z_init.shape[-1]
        P = z_init.numel() // D
        t = self.uncond_transition
        bf16, f32 = torch.bfloat16, torch.float32
        if _ops.fp32_mode(z_init):
            c = lambda x: x.to(f32).contiguous()  # noqa: E731
            out = torch.empty_like(z_init, dtype=f32)
            ws = self._workspace(_ops.trunk_uncond_f32_workspace_bytes(P, D, t.hidden), z_init.device)
            _ops.launch_trunk_uncond_f32(
                c(z_init), c(self.z_norm.weight), c(self.z_norm.bias), c(t.norm.weight), c(t.norm.bias),
                c(t.fc1.weight), c(t.fc2.weight), c(t.fc3.weight), out, ws=ws)
            return s_init, out
        z0, z0_tail = split_stream(z_init)
        ws = self._workspace(_ops.trunk_uncond_workspace_bytes(P, D, t.hidden), z_init.device)
        _ops.launch_trunk_uncond(
            z0, self.z_norm.weight.to(f32).contiguous(), self.z_norm.bias.to(f32).contiguous(),
            t.norm.weight.to(f32).contiguous(), t.norm.bias.to(f32).contiguous(), t.fc1.weight.to(bf16).contiguous(),
            t.fc2.weight.to(bf16).contiguous(), t.fc3.weight.to(bf16).contiguous(), z0, z_init_tail=z0_tail,
            out_tail=z0_tail, ws=ws)
        return s_init, join_stream(z0, z0_tail, z_init.dtype)

    @torch.no_grad()
    def forward(self, s_init: Tensor, z_init: Tensor, s_inputs: Tensor, feats: dict,
                num_steps_recycle: int = 0, unconditional: bool = False) -> tuple[Tensor, Tensor]:
        if not unconditional and num_steps_recycle < 0:
            raise ValueError("num_steps_recycle must be non-negative; use unconditional=True.")
        if unconditional:
            return self.forward_unconditional(s_init, z_init)
        _ops.require_gpu(z_init, type(self).__name__)
        if _ops.fp32_mode(z_init):
            return self._forward_f32(s_init, z_init, s_inputs, feats, num_steps_recycle)
        B, N = z_init.shape[:2]
        S = feats["msa"].shape[1]
        ws = self._workspace(self.workspace_bytes(B, S, N, s_init.shape[-1]), z_init.device)
        bf16 = torch.bfloat16
        (s0, s0_tail), (z0, z0_tail) = split_stream(s_init), split_stream(z_init)
        s, s_tail = torch.zeros_like(s0), torch.zeros_like(s0_tail)   # :257-258
        z, z_tail = torch.zeros_like(z0), torch.zeros_like(z0_tail)
        tok = feats["token_pad_mask"].bool()
        pm = tok[:, :, None] & tok[:, None, :]                          # :263-264
        f32 = torch.float32
        norm = lambda m: (m.weight.to(f32).contiguous(), m.bias.to(f32).contiguous())  # noqa: E731
        w_s, w_z = self.s_recycle.weight.to(bf16).contiguous(), self.z_recycle.weight.to(bf16).contiguous()
        for _ in range(num_steps_recycle + 1):                          # :275
            _ops.launch_ln_linear(s, *norm(self.s_norm), w_s, s0, s, base_tail=s0_tail, out_tail=s_tail, ws=ws)
            _ops.launch_ln_linear(z, *norm(self.z_norm), w_z, z0, z, base_tail=z0_tail, out_tail=z_tail, ws=ws)
            self.msa_module.forward_(z, s_inputs, feats["msa"], feats["msa_mask"], feats["has_deletion"],
                                     feats["deletion_value"], feats.get("msa_paired"), feats["token_pad_mask"],
                                     z_tail, ws=ws)                     # :284-294
            self.pairmixer_module.forward_(s, z, pm, z_tail, ws=ws)    # :296
        return join_stream(s, s_tail, s_init.dtype), join_stream(z, z_tail, z_init.dtype)

    def _forward_f32(self, s_init: Tensor, z_init: Tensor, s_inputs: Tensor, feats: dict,
                     num_steps_recycle: int) -> tuple[Tensor, Tensor]:
        """The recycling loop of :275-296 in IEEE fp32 (autocast off): fp32 s and z, fp32 recycling updates,
        the MSA module's and the PairMixer layers' fp32 paths."""
        B, N = z_init.shape[:2]
        S = feats["msa"].shape[1]
        f32 = torch.float32
        ws = self._workspace(self.workspace_bytes_f32(B, S, N, s_init.shape[-1]), z_init.device)
        s0, z0 = s_init.to(f32).contiguous(), z_init.to(f32).contiguous()
        s, z = torch.zeros_like(s0), torch.zeros_like(z0)                 # :257-258
        tok = feats["token_pad_mask"].bool()
        pm = tok[:, :, None] & tok[:, None, :]                            # :263-264
        c = lambda x: x.to(f32).contiguous()  # noqa: E731
        for _ in range(num_steps_recycle + 1):                            # :275
            _ops.launch_ln_linear_f32(s, c(self.s_norm.weight), c(self.s_norm.bias), c(self.s_recycle.weight), s0, s,
                                      ws=ws)
            _ops.launch_ln_linear_f32(z, c(self.z_norm.weight), c(self.z_norm.bias), c(self.z_recycle.weight), z0, z,
                                      ws=ws)
            self.msa_module.forward_f32_(z, s_inputs, feats["msa"], feats["msa_mask"], feats["has_deletion"],
                                         feats["deletion_value"], feats.get("msa_paired"), feats["token_pad_mask"],
                                         ws=ws)                            # :284-294
            for layer in self.pairmixer_module.layers:                     # :296 (pairmixer.py:368-369)
                layer.forward_f32_(s, z, pm, ws=ws)
        return s, z
