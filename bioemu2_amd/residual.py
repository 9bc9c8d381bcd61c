"""Residual streams carried as (bf16 value, int8 tail).

A stream element's value is ``hi + t * 2**(E(hi) - 142)``: ``hi`` the bf16
element, ``E`` its biased exponent field and ``t`` the int8 tail, i.e. 1/256ths
of hi's unit in the last place, ~16 significant bits in total.  The HIP ops
that add into a stream (``residual=True``) read value + tail and write back a
new (hi, tail), so a stack of ops rounds the stream once, when it is joined.
The reference's bf16-autocast trunk instead stores the stream in bf16 and rounds
it after every add (bf16 z + bf16 update, src/bioemu2/biomoa/modules/
pairmixer.py:446-456, model.py:216-223).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _ops


def split_stream(x: Tensor) -> tuple[Tensor, Tensor]:
    """A new residual stream (bf16 value, int8 tail) holding ``x`` (fp32 or bf16, on the GPU)."""
    _ops.require_gpu(x, "split_stream")
    if x.dtype == torch.bfloat16:
        return x.contiguous().clone(), torch.zeros(x.shape, dtype=torch.int8, device=x.device)
    return _ops.stream_split(x.to(torch.float32).contiguous())


def join_stream(hi: Tensor, tail: Tensor, dtype: torch.dtype = torch.float32) -> Tensor:
    """The stream's value in ``dtype``: fp32 exactly (hi + tail), other dtypes rounded once from it.

    For bf16 that rounding is ``hi`` itself: hi is the nearest bf16 of the value and the tail is at most
    127/256 of its ulp, less than half, so rounding hi + tail to bf16 gives hi back (bit for bit, except
    that a -0 stays -0 where the fp32 sum -0 + 0 is +0), and ``hi`` is returned without another pass over
    the stream."""
    if dtype == torch.bfloat16:
        return hi
    full = _ops.stream_join(hi, tail)
    return full if dtype == torch.float32 else full.to(dtype)
