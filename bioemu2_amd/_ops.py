"""torch ops over the C ABI: ``torch.ops.bioemu_mi355x.*``.

Two layers:

* ``launch_*`` functions: validate tensors and call the C ABI on the current
  HIP stream with caller-provided outputs (no allocation besides the
  workspace).  The Pairformer block uses these directly (with residual fusion).
* ``torch.library`` custom ops (namespace ``bioemu_mi355x``) that allocate
  their output; the drop-in ``nn.Module`` classes call these.

All ops are registered for the CUDA (HIP) device only: a CPU tensor raises,
there is no CPU fallback.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from ._lib import check, lib

BF16 = torch.bfloat16


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(t: Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{what}: bioemu2_amd kernels run on a ROCm GPU only (tensor on {t.device}); "
            "there is no CPU path"
        )


def _check_tensor(t: Tensor, what: str, dtype: torch.dtype, shape: tuple[int, ...], device) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{what}: expected dtype {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{what}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    if t.device != device:
        raise ValueError(f"{what}: tensor on {t.device}, expected {device}")


def mask_u8(mask: Tensor) -> Tensor:
    """Reference masks are bool or 0/1 numbers; nonzero = valid (``mask.bool()``)."""
    if mask.dtype == torch.bool:
        return mask.contiguous().view(torch.uint8)
    return mask.ne(0).contiguous().view(torch.uint8)


def workspace(nbytes: int, device) -> Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


# ----------------------------------------------------------------------------
# Triangle multiplication
# ----------------------------------------------------------------------------
def trimul_workspace_bytes(B: int, N: int, D: int) -> int:
    return int(lib().bioemu_trimul_workspace_bytes(B, N, D))


def launch_trimul(
    x: Tensor,
    mask: Tensor,
    norm_in_w: Tensor,
    norm_in_b: Tensor,
    p_in_w: Tensor,
    g_in_w: Tensor,
    norm_out_w: Tensor,
    norm_out_b: Tensor,
    p_out_w: Tensor,
    g_out_w: Tensor,
    out: Tensor,
    outgoing: bool,
    residual: bool = False,
    ws: Tensor | None = None,
) -> Tensor:
    require_gpu(x, "trimul")
    if x.ndim != 4 or x.shape[1] != x.shape[2]:
        raise ValueError(f"trimul: x must be [B,N,N,D], got {tuple(x.shape)}")
    B, N, _, D = x.shape
    dev = x.device
    _check_tensor(x, "trimul x", BF16, (B, N, N, D), dev)
    _check_tensor(out, "trimul out", BF16, (B, N, N, D), dev)
    _check_tensor(mask, "trimul mask", torch.uint8, (B, N, N), dev)
    for name, t, shp, dt in (
        ("norm_in.weight", norm_in_w, (D,), torch.float32),
        ("norm_in.bias", norm_in_b, (D,), torch.float32),
        ("p_in.weight", p_in_w, (2 * D, D), BF16),
        ("g_in.weight", g_in_w, (2 * D, D), BF16),
        ("norm_out.weight", norm_out_w, (D,), torch.float32),
        ("norm_out.bias", norm_out_b, (D,), torch.float32),
        ("p_out.weight", p_out_w, (D, D), BF16),
        ("g_out.weight", g_out_w, (D, D), BF16),
    ):
        _check_tensor(t, f"trimul {name}", dt, shp, dev)
    need = trimul_workspace_bytes(B, N, D)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_trimul_fwd(
        _ptr(x), _ptr(mask), _ptr(norm_in_w), _ptr(norm_in_b), _ptr(p_in_w), _ptr(g_in_w),
        _ptr(norm_out_w), _ptr(norm_out_b), _ptr(p_out_w), _ptr(g_out_w), _ptr(out),
        _ptr(ws), ctypes.c_size_t(ws.numel()), B, N, D, int(bool(outgoing)), int(bool(residual)),
        _stream(x),
    )
    check(rc, "bioemu_trimul_fwd")
    return out


@torch.library.custom_op("bioemu_mi355x::trimul", mutates_args=(), device_types="cuda")
def trimul(
    x: Tensor,
    mask: Tensor,
    norm_in_w: Tensor,
    norm_in_b: Tensor,
    p_in_w: Tensor,
    g_in_w: Tensor,
    norm_out_w: Tensor,
    norm_out_b: Tensor,
    p_out_w: Tensor,
    g_out_w: Tensor,
    outgoing: bool,
) -> Tensor:
    xb = x.to(BF16).contiguous()
    out = torch.empty_like(xb)
    f32 = torch.float32
    launch_trimul(
        xb, mask_u8(mask), norm_in_w.to(f32).contiguous(), norm_in_b.to(f32).contiguous(),
        p_in_w.to(BF16).contiguous(), g_in_w.to(BF16).contiguous(),
        norm_out_w.to(f32).contiguous(), norm_out_b.to(f32).contiguous(),
        p_out_w.to(BF16).contiguous(), g_out_w.to(BF16).contiguous(), out, outgoing,
    )
    return out.to(x.dtype)


@trimul.register_fake
def _(x, mask, norm_in_w, norm_in_b, p_in_w, g_in_w, norm_out_w, norm_out_b, p_out_w, g_out_w, outgoing):
    return torch.empty_like(x)


# ----------------------------------------------------------------------------
# Triangle attention
# ----------------------------------------------------------------------------
def triatt_workspace_bytes(B: int, N: int, D: int = 128, H: int = 4) -> int:
    return int(lib().bioemu_triatt_workspace_bytes(B, N, D, H))


def launch_triatt(
    z: Tensor,
    mask: Tensor,
    norm_w: Tensor,
    norm_b: Tensor,
    w_proj: Tensor,
    w_o: Tensor,
    out: Tensor,
    starting: bool,
    num_heads: int = 4,
    residual: bool = False,
    ws: Tensor | None = None,
) -> Tensor:
    require_gpu(z, "triatt")
    if z.ndim != 4 or z.shape[1] != z.shape[2]:
        raise ValueError(f"triatt: z must be [B,N,N,D], got {tuple(z.shape)}")
    B, N, _, D = z.shape
    dev = z.device
    _check_tensor(z, "triatt z", BF16, (B, N, N, D), dev)
    _check_tensor(out, "triatt out", BF16, (B, N, N, D), dev)
    _check_tensor(mask, "triatt mask", torch.uint8, (B, N, N), dev)
    _check_tensor(norm_w, "triatt norm.weight", torch.float32, (D,), dev)
    _check_tensor(norm_b, "triatt norm.bias", torch.float32, (D,), dev)
    _check_tensor(w_proj, "triatt packed projection", BF16, (4 * D + num_heads, D), dev)
    _check_tensor(w_o, "triatt proj_o.weight", BF16, (D, D), dev)
    need = triatt_workspace_bytes(B, N, D, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_triatt_fwd(
        _ptr(z), _ptr(mask), _ptr(norm_w), _ptr(norm_b), _ptr(w_proj), _ptr(w_o), _ptr(out),
        _ptr(ws), ctypes.c_size_t(ws.numel()), B, N, D, num_heads, int(bool(starting)),
        int(bool(residual)), _stream(z),
    )
    check(rc, "bioemu_triatt_fwd")
    return out


@torch.library.custom_op("bioemu_mi355x::triangle_attention", mutates_args=(), device_types="cuda")
def triangle_attention(
    z: Tensor,
    mask: Tensor,
    norm_w: Tensor,
    norm_b: Tensor,
    w_proj: Tensor,
    w_o: Tensor,
    starting: bool,
    num_heads: int,
) -> Tensor:
    zb = z.to(BF16).contiguous()
    out = torch.empty_like(zb)
    f32 = torch.float32
    launch_triatt(
        zb, mask_u8(mask), norm_w.to(f32).contiguous(), norm_b.to(f32).contiguous(),
        w_proj.to(BF16).contiguous(), w_o.to(BF16).contiguous(), out, starting, num_heads,
    )
    return out.to(z.dtype)


@triangle_attention.register_fake
def _(z, mask, norm_w, norm_b, w_proj, w_o, starting, num_heads):
    return torch.empty_like(z)
