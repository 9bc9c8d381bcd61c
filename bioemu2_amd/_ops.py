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
F32 = torch.float32


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


def _check_tail(tail: Tensor | None, out: Tensor, residual: bool, what: str) -> None:
    """A residual tail is the int8 plane of the stream ``out`` is written into (one byte per element)."""
    if tail is None:
        return
    if not residual:
        raise ValueError(f"{what}: a residual tail needs residual=True")
    _check_tensor(tail, f"{what} residual tail", torch.int8, tuple(out.shape), out.device)


# ----------------------------------------------------------------------------
# Residual streams: fp32 <-> (bf16 value, int8 tail)
# ----------------------------------------------------------------------------
def stream_split(x: Tensor, hi: Tensor | None = None, tail: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """fp32 ``x`` -> (bf16 ``hi``, int8 ``tail``) with hi + tail carrying ~16 significant bits."""
    require_gpu(x, "stream_split")
    if x.dtype != torch.float32 or not x.is_contiguous() or x.numel() % 16:
        raise ValueError("stream_split: x must be a contiguous fp32 tensor with a multiple of 16 elements")
    hi = torch.empty(x.shape, dtype=BF16, device=x.device) if hi is None else hi
    tail = torch.empty(x.shape, dtype=torch.int8, device=x.device) if tail is None else tail
    _check_tensor(hi, "stream_split hi", BF16, tuple(x.shape), x.device)
    _check_tensor(tail, "stream_split tail", torch.int8, tuple(x.shape), x.device)
    check(lib().bioemu_stream_split(_ptr(x), _ptr(hi), _ptr(tail), x.numel(), _stream(x)), "bioemu_stream_split")
    return hi, tail


def stream_join(hi: Tensor, tail: Tensor, out: Tensor | None = None) -> Tensor:
    """(bf16 ``hi``, int8 ``tail``) -> fp32."""
    require_gpu(hi, "stream_join")
    if hi.numel() % 16:
        raise ValueError("stream_join: element count must be a multiple of 16")
    _check_tensor(hi, "stream_join hi", BF16, tuple(hi.shape), hi.device)
    _check_tensor(tail, "stream_join tail", torch.int8, tuple(hi.shape), hi.device)
    out = torch.empty(hi.shape, dtype=torch.float32, device=hi.device) if out is None else out
    _check_tensor(out, "stream_join out", torch.float32, tuple(hi.shape), hi.device)
    check(lib().bioemu_stream_join(_ptr(hi), _ptr(tail), _ptr(out), hi.numel(), _stream(hi)), "bioemu_stream_join")
    return out


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
    tail: Tensor | None = None,
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
    _check_tail(tail, out, residual, "trimul")
    need = trimul_workspace_bytes(B, N, D)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_trimul_fwd(
        _ptr(x), _ptr(mask), _ptr(norm_in_w), _ptr(norm_in_b), _ptr(p_in_w), _ptr(g_in_w),
        _ptr(norm_out_w), _ptr(norm_out_b), _ptr(p_out_w), _ptr(g_out_w), _ptr(out), _ptr(tail),
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


def trimul_f32_workspace_bytes(B: int, N: int, D: int) -> int:
    return int(lib().bioemu_trimul_f32_workspace_bytes(B, N, D))


def launch_trimul_f32(
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
    """The triangle multiplicative update in IEEE fp32 (``bioemu_trimul_fwd_f32``): every tensor fp32."""
    require_gpu(x, "trimul_f32")
    if x.ndim != 4 or x.shape[1] != x.shape[2]:
        raise ValueError(f"trimul_f32: x must be [B,N,N,D], got {tuple(x.shape)}")
    B, N, _, D = x.shape
    dev = x.device
    _check_tensor(x, "trimul_f32 x", F32, (B, N, N, D), dev)
    _check_tensor(out, "trimul_f32 out", F32, (B, N, N, D), dev)
    _check_tensor(mask, "trimul_f32 mask", torch.uint8, (B, N, N), dev)
    for name, t, shp in (
        ("norm_in.weight", norm_in_w, (D,)), ("norm_in.bias", norm_in_b, (D,)),
        ("p_in.weight", p_in_w, (2 * D, D)), ("g_in.weight", g_in_w, (2 * D, D)),
        ("norm_out.weight", norm_out_w, (D,)), ("norm_out.bias", norm_out_b, (D,)),
        ("p_out.weight", p_out_w, (D, D)), ("g_out.weight", g_out_w, (D, D)),
    ):
        _check_tensor(t, f"trimul_f32 {name}", F32, shp, dev)
    need = trimul_f32_workspace_bytes(B, N, D)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_trimul_fwd_f32(
        _ptr(x), _ptr(mask), _ptr(norm_in_w), _ptr(norm_in_b), _ptr(p_in_w), _ptr(g_in_w),
        _ptr(norm_out_w), _ptr(norm_out_b), _ptr(p_out_w), _ptr(g_out_w), _ptr(out),
        _ptr(ws), ctypes.c_size_t(ws.numel()), B, N, D, int(bool(outgoing)), int(bool(residual)), _stream(x),
    )
    check(rc, "bioemu_trimul_fwd_f32")
    return out


@torch.library.custom_op("bioemu_mi355x::trimul_f32", mutates_args=(), device_types="cuda")
def trimul_f32(
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
    xf = x.contiguous()
    out = torch.empty_like(xf)
    f32c = lambda t: t.to(F32).contiguous()  # noqa: E731
    launch_trimul_f32(xf, mask_u8(mask), f32c(norm_in_w), f32c(norm_in_b), f32c(p_in_w), f32c(g_in_w),
                      f32c(norm_out_w), f32c(norm_out_b), f32c(p_out_w), f32c(g_out_w), out, outgoing)
    return out


@trimul_f32.register_fake
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
    tail: Tensor | None = None,
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
    _check_tail(tail, out, residual, "triatt")
    need = triatt_workspace_bytes(B, N, D, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_triatt_fwd(
        _ptr(z), _ptr(mask), _ptr(norm_w), _ptr(norm_b), _ptr(w_proj), _ptr(w_o), _ptr(out), _ptr(tail),
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


def triatt_f32_workspace_bytes(B: int, N: int, D: int = 128, H: int = 4) -> int:
    return int(lib().bioemu_triatt_f32_workspace_bytes(B, N, D, H))


def launch_triatt_f32(
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
    """Triangle attention in fp32 (``bioemu_triatt_fwd_f32``): the arguments of ``launch_triatt``, every
    tensor fp32 (the mask uint8), no tail."""
    require_gpu(z, "triatt_f32")
    if z.ndim != 4 or z.shape[1] != z.shape[2]:
        raise ValueError(f"triatt_f32: z must be [B,N,N,D], got {tuple(z.shape)}")
    B, N, _, D = z.shape
    dev = z.device
    _check_tensor(z, "triatt_f32 z", F32, (B, N, N, D), dev)
    _check_tensor(out, "triatt_f32 out", F32, (B, N, N, D), dev)
    _check_tensor(mask, "triatt_f32 mask", torch.uint8, (B, N, N), dev)
    _check_tensor(norm_w, "triatt_f32 norm.weight", F32, (D,), dev)
    _check_tensor(norm_b, "triatt_f32 norm.bias", F32, (D,), dev)
    _check_tensor(w_proj, "triatt_f32 packed projection", F32, (4 * D + num_heads, D), dev)
    _check_tensor(w_o, "triatt_f32 proj_o.weight", F32, (D, D), dev)
    need = triatt_f32_workspace_bytes(B, N, D, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_triatt_fwd_f32(
        _ptr(z), _ptr(mask), _ptr(norm_w), _ptr(norm_b), _ptr(w_proj), _ptr(w_o), _ptr(out), _ptr(ws),
        ctypes.c_size_t(ws.numel()), B, N, D, num_heads, int(bool(starting)), int(bool(residual)), _stream(z),
    )
    check(rc, "bioemu_triatt_fwd_f32")
    return out


@torch.library.custom_op("bioemu_mi355x::triangle_attention_f32", mutates_args=(), device_types="cuda")
def triangle_attention_f32(
    z: Tensor,
    mask: Tensor,
    norm_w: Tensor,
    norm_b: Tensor,
    w_proj: Tensor,
    w_o: Tensor,
    starting: bool,
    num_heads: int,
) -> Tensor:
    zf = z.contiguous()
    out = torch.empty_like(zf)
    f32c = lambda t: t.to(F32).contiguous()  # noqa: E731
    launch_triatt_f32(zf, mask_u8(mask), f32c(norm_w), f32c(norm_b), f32c(w_proj), f32c(w_o), out, starting,
                      num_heads)
    return out


@triangle_attention_f32.register_fake
def _(z, mask, norm_w, norm_b, w_proj, w_o, starting, num_heads):
    return torch.empty_like(z)


# ----------------------------------------------------------------------------
# Transition (SwiGLU MLP)
# ----------------------------------------------------------------------------
def transition_pair_workspace_bytes(D: int, hidden: int) -> int:
    return int(lib().bioemu_transition_pair_workspace_bytes(D, hidden))


def launch_transition_pair(
    x: Tensor,
    norm_w: Tensor | None,
    norm_b: Tensor | None,
    fc1_w: Tensor,
    fc2_w: Tensor,
    fc3_w: Tensor,
    out: Tensor,
    residual: bool = False,
    ws: Tensor | None = None,
    tail: Tensor | None = None,
) -> Tensor:
    require_gpu(x, "transition")
    D = x.shape[-1]
    P = x.numel() // D
    dev = x.device
    hidden = fc1_w.shape[0]
    _check_tensor(x, "transition x", BF16, tuple(x.shape), dev)
    _check_tensor(out, "transition out", BF16, tuple(x.shape), dev)
    _check_tensor(fc1_w, "transition fc1.weight", BF16, (hidden, D), dev)
    _check_tensor(fc2_w, "transition fc2.weight", BF16, (hidden, D), dev)
    _check_tensor(fc3_w, "transition fc3.weight", BF16, (D, hidden), dev)
    use_norm = norm_w is not None
    if use_norm:
        _check_tensor(norm_w, "transition norm.weight", torch.float32, (D,), dev)
        _check_tensor(norm_b, "transition norm.bias", torch.float32, (D,), dev)
    _check_tail(tail, out, residual, "transition")
    need = transition_pair_workspace_bytes(D, hidden)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_transition_pair_fwd(
        _ptr(x), _ptr(norm_w), _ptr(norm_b), _ptr(fc1_w), _ptr(fc2_w), _ptr(fc3_w), _ptr(out), _ptr(tail),
        _ptr(ws), ctypes.c_size_t(ws.numel()), P, D, hidden, int(use_norm), int(bool(residual)), _stream(x),
    )
    check(rc, "bioemu_transition_pair_fwd")
    return out


def transition_token_workspace_bytes(M: int, D: int, hidden: int) -> int:
    return int(lib().bioemu_transition_token_workspace_bytes(M, D, hidden))


def launch_transition_token(
    x: Tensor,
    norm_w: Tensor | None,
    norm_b: Tensor | None,
    fc1_w: Tensor,
    fc2_w: Tensor,
    fc3_w: Tensor,
    out: Tensor,
    residual: bool = False,
    ws: Tensor | None = None,
    tail: Tensor | None = None,
) -> Tensor:
    require_gpu(x, "transition")
    D = x.shape[-1]
    M = x.numel() // D
    dev = x.device
    hidden = fc1_w.shape[0]
    out_dim = fc3_w.shape[0]
    _check_tensor(x, "transition x", BF16, tuple(x.shape), dev)
    _check_tensor(out, "transition out", BF16, tuple(x.shape[:-1]) + (out_dim,), dev)
    _check_tensor(fc1_w, "transition fc1.weight", BF16, (hidden, D), dev)
    _check_tensor(fc2_w, "transition fc2.weight", BF16, (hidden, D), dev)
    _check_tensor(fc3_w, "transition fc3.weight", BF16, (out_dim, hidden), dev)
    use_norm = norm_w is not None
    if use_norm:
        _check_tensor(norm_w, "transition norm.weight", torch.float32, (D,), dev)
        _check_tensor(norm_b, "transition norm.bias", torch.float32, (D,), dev)
    _check_tail(tail, out, residual, "transition")
    need = transition_token_workspace_bytes(M, D, hidden)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_transition_token_fwd(
        _ptr(x), _ptr(norm_w), _ptr(norm_b), _ptr(fc1_w), _ptr(fc2_w), _ptr(fc3_w), _ptr(out), _ptr(tail),
        _ptr(ws), ctypes.c_size_t(ws.numel()), M, D, hidden, out_dim, int(use_norm), int(bool(residual)),
        _stream(x),
    )
    check(rc, "bioemu_transition_token_fwd")
    return out


def _is_row_transition(x: Tensor, hidden: int) -> bool:
    """Widths the fused row kernel takes: rows of 64 or 128 channels with hidden 4x (the trunk's pair and MSA
    transitions) or 2x (the denoiser's pairwise conditioning)."""
    return x.shape[-1] in (64, 128) and hidden in (2 * x.shape[-1], 4 * x.shape[-1])


@torch.library.custom_op("bioemu_mi355x::transition", mutates_args=(), device_types="cuda")
def transition(
    x: Tensor, norm_w: Tensor | None, norm_b: Tensor | None, fc1_w: Tensor, fc2_w: Tensor, fc3_w: Tensor
) -> Tensor:
    xb = x.to(BF16).contiguous()
    out_dim = fc3_w.shape[0]
    out = torch.empty(*xb.shape[:-1], out_dim, dtype=BF16, device=xb.device)
    f32 = torch.float32
    nw = None if norm_w is None else norm_w.to(f32).contiguous()
    nb = None if norm_b is None else norm_b.to(f32).contiguous()
    w1, w2, w3 = (w.to(BF16).contiguous() for w in (fc1_w, fc2_w, fc3_w))
    if out_dim == xb.shape[-1] and _is_row_transition(xb, w1.shape[0]):
        launch_transition_pair(xb, nw, nb, w1, w2, w3, out)
    else:
        launch_transition_token(xb, nw, nb, w1, w2, w3, out)
    return out.to(x.dtype)


@transition.register_fake
def _(x, norm_w, norm_b, fc1_w, fc2_w, fc3_w):
    return x.new_empty(*x.shape[:-1], fc3_w.shape[0])


# ----------------------------------------------------------------------------
# Attention with pair bias
# ----------------------------------------------------------------------------
def apb_workspace_bytes(B: int, mult: int, N: int, c_s: int, H: int) -> int:
    return int(lib().bioemu_apb_workspace_bytes(B, mult, N, c_s, H))


def launch_apb(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    out: Tensor,
    num_heads: int,
    multiplicity: int = 1,
    residual: bool = False,
    ws: Tensor | None = None,
    tail: Tensor | None = None,
) -> Tensor:
    require_gpu(s, "attention_pair_bias")
    if s.ndim != 3 or z.ndim != 4 or mask.ndim != 2:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, {tuple(mask.shape)}")
    if s.shape[0] != z.shape[0] * multiplicity:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, multiplicity={multiplicity}")
    BM, N, c_s = s.shape
    B, _, _, c_z = z.shape
    dev = s.device
    _check_tensor(s, "apb s", BF16, (BM, N, c_s), dev)
    _check_tensor(out, "apb out", BF16, (BM, N, c_s), dev)
    _check_tensor(z, "apb z", BF16, (B, N, N, c_z), dev)
    _check_tensor(mask, "apb mask", torch.uint8, (B, N), dev)
    if norm_s_w is not None:
        _check_tensor(norm_s_w, "apb norm_s.weight", torch.float32, (c_s,), dev)
        _check_tensor(norm_s_b, "apb norm_s.bias", torch.float32, (c_s,), dev)
    _check_tensor(w_qkv, "apb proj_qkv.weight", BF16, (3 * c_s, c_s), dev)
    _check_tensor(q_bias, "apb proj_q_bias", torch.float32, (c_s,), dev)
    _check_tensor(w_g, "apb proj_g.weight", BF16, (c_s, c_s), dev)
    _check_tensor(norm_z_w, "apb norm_z.weight", torch.float32, (c_z,), dev)
    if norm_z_b is not None:
        _check_tensor(norm_z_b, "apb norm_z.bias", torch.float32, (c_z,), dev)
    _check_tensor(w_z, "apb proj_z.weight", BF16, (num_heads, c_z), dev)
    _check_tensor(w_o, "apb proj_o.weight", BF16, (c_s, c_s), dev)
    _check_tail(tail, out, residual, "apb")
    need = apb_workspace_bytes(B, multiplicity, N, c_s, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_apb_fwd(
        _ptr(s), _ptr(z), _ptr(mask), _ptr(norm_s_w), _ptr(norm_s_b), _ptr(w_qkv), _ptr(q_bias), _ptr(w_g),
        _ptr(norm_z_w), _ptr(norm_z_b), _ptr(w_z), _ptr(w_o), _ptr(out), _ptr(tail), _ptr(ws),
        ctypes.c_size_t(ws.numel()),
        B, multiplicity, N, c_s, c_z, num_heads, int(bool(residual)), _stream(s),
    )
    check(rc, "bioemu_apb_fwd")
    return out


@torch.library.custom_op("bioemu_mi355x::attention_pair_bias", mutates_args=(), device_types="cuda")
def attention_pair_bias(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    num_heads: int,
    multiplicity: int,
) -> Tensor:
    sb = s.to(BF16).contiguous()
    out = torch.empty_like(sb)
    f32 = torch.float32

    def f(t):
        return None if t is None else t.to(f32).contiguous()

    def h(t):
        return t.to(BF16).contiguous()

    launch_apb(
        sb, h(z), mask_u8(mask), f(norm_s_w), f(norm_s_b), h(w_qkv), f(q_bias), h(w_g), f(norm_z_w), f(norm_z_b),
        h(w_z), h(w_o), out, num_heads, multiplicity,
    )
    return out.to(s.dtype)


@attention_pair_bias.register_fake
def _(s, z, mask, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w, norm_z_b, w_z, w_o, num_heads, multiplicity):
    return torch.empty_like(s)


# ----------------------------------------------------------------------------
# Sliding-window attention with pair bias
# ----------------------------------------------------------------------------
def swa_workspace_bytes(B: int, mult: int, NW: int, W: int, H: int, c_s: int, heads: int) -> int:
    return int(lib().bioemu_swa_workspace_bytes(B, mult, NW, W, H, c_s, heads))


def launch_swa(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    out: Tensor,
    num_heads: int,
    multiplicity: int = 1,
    residual: bool = False,
    ws: Tensor | None = None,
) -> Tensor:
    """s [B*M*NW, W, c_s], z [B, NW, W, H, c_z], mask [B*NW, W] uint8 (attention_pair_bias.py:277-340)."""
    require_gpu(s, "attention_pair_bias_sliding_window")
    if s.ndim != 3 or z.ndim != 5 or mask.ndim != 2:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, {tuple(mask.shape)}")
    B, NW, W, H, c_z = z.shape
    folded, _, c_s = s.shape
    if folded != B * multiplicity * NW:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, multiplicity={multiplicity}")
    dev = s.device
    _check_tensor(s, "swa s", BF16, (folded, W, c_s), dev)
    _check_tensor(out, "swa out", BF16, (folded, W, c_s), dev)
    _check_tensor(z, "swa z", BF16, (B, NW, W, H, c_z), dev)
    _check_tensor(mask, "swa mask", torch.uint8, (B * NW, W), dev)
    if norm_s_w is not None:
        _check_tensor(norm_s_w, "swa norm_s.weight", torch.float32, (c_s,), dev)
        _check_tensor(norm_s_b, "swa norm_s.bias", torch.float32, (c_s,), dev)
    _check_tensor(w_qkv, "swa proj_qkv.weight", BF16, (3 * c_s, c_s), dev)
    _check_tensor(q_bias, "swa proj_q_bias", torch.float32, (c_s,), dev)
    _check_tensor(w_g, "swa proj_g.weight", BF16, (c_s, c_s), dev)
    _check_tensor(norm_z_w, "swa norm_z.weight", torch.float32, (c_z,), dev)
    if norm_z_b is not None:
        _check_tensor(norm_z_b, "swa norm_z.bias", torch.float32, (c_z,), dev)
    _check_tensor(w_z, "swa proj_z.weight", BF16, (num_heads, c_z), dev)
    _check_tensor(w_o, "swa proj_o.weight", BF16, (c_s, c_s), dev)
    need = swa_workspace_bytes(B, multiplicity, NW, W, H, c_s, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_swa_fwd(
        _ptr(s), _ptr(z), _ptr(mask), _ptr(norm_s_w), _ptr(norm_s_b), _ptr(w_qkv), _ptr(q_bias), _ptr(w_g),
        _ptr(norm_z_w), _ptr(norm_z_b), _ptr(w_z), _ptr(w_o), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()),
        B, multiplicity, NW, W, H, c_s, c_z, num_heads, int(bool(residual)), _stream(s),
    )
    check(rc, "bioemu_swa_fwd")
    return out


@torch.library.custom_op("bioemu_mi355x::attention_pair_bias_sliding_window", mutates_args=(), device_types="cuda")
def attention_pair_bias_sliding_window(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    num_heads: int,
    multiplicity: int,
) -> Tensor:
    sb = s.to(BF16).contiguous()
    out = torch.empty_like(sb)
    f32 = torch.float32

    def f(t):
        return None if t is None else t.to(f32).contiguous()

    def h(t):
        return t.to(BF16).contiguous()

    launch_swa(
        sb, h(z), mask_u8(mask), f(norm_s_w), f(norm_s_b), h(w_qkv), f(q_bias), h(w_g), f(norm_z_w), f(norm_z_b),
        h(w_z), h(w_o), out, num_heads, multiplicity,
    )
    return out.to(s.dtype)


@attention_pair_bias_sliding_window.register_fake
def _(s, z, mask, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w, norm_z_b, w_z, w_o, num_heads, multiplicity):
    return torch.empty_like(s)


# ----------------------------------------------------------------------------
# fp32 arithmetic path (the reference's denoiser runs with autocast off)
# ----------------------------------------------------------------------------


def fp32_mode(x: Tensor) -> bool:
    """True where the reference computes in fp32: fp32 inputs with CUDA autocast off.

    The reference's denoiser disables autocast (score_model.py:355, model.py:387), so its attention and
    transitions run fp32 on fp32 activations; under bf16 autocast (the trunk) they run bf16 matmuls.
    """
    return x.dtype == F32 and not torch.is_autocast_enabled("cuda")


def _check_attn_params_f32(what, c_s, c_z, num_heads, dev, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w,
                           norm_z_b, w_z, w_o) -> None:
    if norm_s_w is not None:
        _check_tensor(norm_s_w, f"{what} norm_s.weight", F32, (c_s,), dev)
        _check_tensor(norm_s_b, f"{what} norm_s.bias", F32, (c_s,), dev)
    _check_tensor(w_qkv, f"{what} proj_qkv.weight", F32, (3 * c_s, c_s), dev)
    _check_tensor(q_bias, f"{what} proj_q_bias", F32, (c_s,), dev)
    _check_tensor(w_g, f"{what} proj_g.weight", F32, (c_s, c_s), dev)
    _check_tensor(norm_z_w, f"{what} norm_z.weight", F32, (c_z,), dev)
    if norm_z_b is not None:
        _check_tensor(norm_z_b, f"{what} norm_z.bias", F32, (c_z,), dev)
    _check_tensor(w_z, f"{what} proj_z.weight", F32, (num_heads, c_z), dev)
    _check_tensor(w_o, f"{what} proj_o.weight", F32, (c_s, c_s), dev)


def apb_f32_workspace_bytes(B: int, mult: int, N: int, c_s: int, H: int) -> int:
    return int(lib().bioemu_apb_f32_workspace_bytes(B, mult, N, c_s, H))


def launch_apb_f32(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    out: Tensor,
    num_heads: int,
    multiplicity: int = 1,
    residual: bool = False,
    ws: Tensor | None = None,
) -> Tensor:
    """fp32 AttentionPairBias (attention_pair_bias.py:128-225): every tensor fp32, mask [B,N] uint8."""
    require_gpu(s, "attention_pair_bias_f32")
    if s.ndim != 3 or z.ndim != 4 or mask.ndim != 2:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, {tuple(mask.shape)}")
    if s.shape[0] != z.shape[0] * multiplicity:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, multiplicity={multiplicity}")
    BM, N, c_s = s.shape
    B, _, _, c_z = z.shape
    dev = s.device
    _check_tensor(s, "apb_f32 s", F32, (BM, N, c_s), dev)
    _check_tensor(out, "apb_f32 out", F32, (BM, N, c_s), dev)
    _check_tensor(z, "apb_f32 z", F32, (B, N, N, c_z), dev)
    _check_tensor(mask, "apb_f32 mask", torch.uint8, (B, N), dev)
    _check_attn_params_f32("apb_f32", c_s, c_z, num_heads, dev, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w,
                           norm_z_b, w_z, w_o)
    need = apb_f32_workspace_bytes(B, multiplicity, N, c_s, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_apb_fwd_f32(
        _ptr(s), _ptr(z), _ptr(mask), _ptr(norm_s_w), _ptr(norm_s_b), _ptr(w_qkv), _ptr(q_bias), _ptr(w_g),
        _ptr(norm_z_w), _ptr(norm_z_b), _ptr(w_z), _ptr(w_o), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()),
        B, multiplicity, N, c_s, c_z, num_heads, int(bool(residual)), _stream(s),
    )
    check(rc, "bioemu_apb_fwd_f32")
    return out


def _f32c(t: Tensor | None) -> Tensor | None:
    return None if t is None else t.to(F32).contiguous()


@torch.library.custom_op("bioemu_mi355x::attention_pair_bias_f32", mutates_args=(), device_types="cuda")
def attention_pair_bias_f32(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    num_heads: int,
    multiplicity: int,
) -> Tensor:
    sf = s.to(F32).contiguous()
    out = torch.empty_like(sf)
    launch_apb_f32(
        sf, _f32c(z), mask_u8(mask), _f32c(norm_s_w), _f32c(norm_s_b), _f32c(w_qkv), _f32c(q_bias), _f32c(w_g),
        _f32c(norm_z_w), _f32c(norm_z_b), _f32c(w_z), _f32c(w_o), out, num_heads, multiplicity,
    )
    return out.to(s.dtype)


@attention_pair_bias_f32.register_fake
def _(s, z, mask, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w, norm_z_b, w_z, w_o, num_heads, multiplicity):
    return torch.empty_like(s)


def swa_f32_workspace_bytes(B: int, mult: int, NW: int, W: int, H: int, c_s: int, heads: int) -> int:
    return int(lib().bioemu_swa_f32_workspace_bytes(B, mult, NW, W, H, c_s, heads))


def launch_swa_f32(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    out: Tensor,
    num_heads: int,
    multiplicity: int = 1,
    residual: bool = False,
    ws: Tensor | None = None,
) -> Tensor:
    """fp32 sliding-window attention (attention_pair_bias.py:277-340): s [B*M*NW, W, c_s], z [B, NW, W, H, c_z],
    mask [B*NW, W] uint8, every other tensor fp32."""
    require_gpu(s, "attention_pair_bias_sliding_window_f32")
    if s.ndim != 3 or z.ndim != 5 or mask.ndim != 2:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, {tuple(mask.shape)}")
    B, NW, W, H, c_z = z.shape
    folded, _, c_s = s.shape
    if folded != B * multiplicity * NW:
        raise AssertionError(f"{tuple(s.shape)}, {tuple(z.shape)}, multiplicity={multiplicity}")
    dev = s.device
    _check_tensor(s, "swa_f32 s", F32, (folded, W, c_s), dev)
    _check_tensor(out, "swa_f32 out", F32, (folded, W, c_s), dev)
    _check_tensor(z, "swa_f32 z", F32, (B, NW, W, H, c_z), dev)
    _check_tensor(mask, "swa_f32 mask", torch.uint8, (B * NW, W), dev)
    if mask.data_ptr() % 4:   # the kernel reads the mask 4 keys at a time
        mask = mask.clone()
    _check_attn_params_f32("swa_f32", c_s, c_z, num_heads, dev, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w,
                           norm_z_b, w_z, w_o)
    need = swa_f32_workspace_bytes(B, multiplicity, NW, W, H, c_s, num_heads)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_swa_fwd_f32(
        _ptr(s), _ptr(z), _ptr(mask), _ptr(norm_s_w), _ptr(norm_s_b), _ptr(w_qkv), _ptr(q_bias), _ptr(w_g),
        _ptr(norm_z_w), _ptr(norm_z_b), _ptr(w_z), _ptr(w_o), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()),
        B, multiplicity, NW, W, H, c_s, c_z, num_heads, int(bool(residual)), _stream(s),
    )
    check(rc, "bioemu_swa_fwd_f32")
    return out


@torch.library.custom_op(
    "bioemu_mi355x::attention_pair_bias_sliding_window_f32", mutates_args=(), device_types="cuda"
)
def attention_pair_bias_sliding_window_f32(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_s_w: Tensor | None,
    norm_s_b: Tensor | None,
    w_qkv: Tensor,
    q_bias: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    num_heads: int,
    multiplicity: int,
) -> Tensor:
    sf = s.to(F32).contiguous()
    out = torch.empty_like(sf)
    launch_swa_f32(
        sf, _f32c(z), mask_u8(mask), _f32c(norm_s_w), _f32c(norm_s_b), _f32c(w_qkv), _f32c(q_bias), _f32c(w_g),
        _f32c(norm_z_w), _f32c(norm_z_b), _f32c(w_z), _f32c(w_o), out, num_heads, multiplicity,
    )
    return out.to(s.dtype)


@attention_pair_bias_sliding_window_f32.register_fake
def _(s, z, mask, norm_s_w, norm_s_b, w_qkv, q_bias, w_g, norm_z_w, norm_z_b, w_z, w_o, num_heads, multiplicity):
    return torch.empty_like(s)


def transition_f32_workspace_bytes(M: int, D: int, hidden: int) -> int:
    return int(lib().bioemu_transition_f32_workspace_bytes(M, D, hidden))


def launch_transition_f32(
    x: Tensor,
    norm_w: Tensor | None,
    norm_b: Tensor | None,
    fc1_w: Tensor,
    fc2_w: Tensor,
    fc3_w: Tensor,
    out: Tensor,
    residual: bool = False,
    ws: Tensor | None = None,
) -> Tensor:
    """fp32 Transition (transition.py:52-76) over the rows of x [..., D]; out [..., out_dim]."""
    require_gpu(x, "transition_f32")
    D = x.shape[-1]
    M = x.numel() // D
    dev = x.device
    hidden = fc1_w.shape[0]
    out_dim = fc3_w.shape[0]
    _check_tensor(x, "transition_f32 x", F32, tuple(x.shape), dev)
    _check_tensor(out, "transition_f32 out", F32, tuple(x.shape[:-1]) + (out_dim,), dev)
    _check_tensor(fc1_w, "transition_f32 fc1.weight", F32, (hidden, D), dev)
    _check_tensor(fc2_w, "transition_f32 fc2.weight", F32, (hidden, D), dev)
    _check_tensor(fc3_w, "transition_f32 fc3.weight", F32, (out_dim, hidden), dev)
    use_norm = norm_w is not None
    if use_norm:
        _check_tensor(norm_w, "transition_f32 norm.weight", F32, (D,), dev)
        _check_tensor(norm_b, "transition_f32 norm.bias", F32, (D,), dev)
    need = transition_f32_workspace_bytes(M, D, hidden)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_transition_fwd_f32(
        _ptr(x), _ptr(norm_w), _ptr(norm_b), _ptr(fc1_w), _ptr(fc2_w), _ptr(fc3_w), _ptr(out), _ptr(ws),
        ctypes.c_size_t(ws.numel()), M, D, hidden, out_dim, int(use_norm), int(bool(residual)), _stream(x),
    )
    check(rc, "bioemu_transition_fwd_f32")
    return out


@torch.library.custom_op("bioemu_mi355x::transition_f32", mutates_args=(), device_types="cuda")
def transition_f32(
    x: Tensor, norm_w: Tensor | None, norm_b: Tensor | None, fc1_w: Tensor, fc2_w: Tensor, fc3_w: Tensor
) -> Tensor:
    xf = x.to(F32).contiguous()
    out = torch.empty(*xf.shape[:-1], fc3_w.shape[0], dtype=F32, device=xf.device)
    launch_transition_f32(xf, _f32c(norm_w), _f32c(norm_b), _f32c(fc1_w), _f32c(fc2_w), _f32c(fc3_w), out)
    return out.to(x.dtype)


@transition_f32.register_fake
def _(x, norm_w, norm_b, fc1_w, fc2_w, fc3_w):
    return x.new_empty(*x.shape[:-1], fc3_w.shape[0])


def pair_cond_f32_workspace_bytes(P: int, token_z: int, c_rel: int) -> int:
    return int(lib().bioemu_pair_cond_f32_workspace_bytes(P, token_z, c_rel))


def launch_pair_cond_proj_f32(
    z_trunk: Tensor, rel: Tensor, ln_w: Tensor, ln_b: Tensor, w: Tensor, out: Tensor, ws: Tensor | None = None
) -> Tensor:
    """fp32 LayerNorm over [z_trunk | rel] + LinearNoBias (PairwiseConditioning, diffusion.py:521-524)."""
    require_gpu(z_trunk, "pair_cond_f32")
    token_z, c_rel = z_trunk.shape[-1], rel.shape[-1]
    lead = tuple(z_trunk.shape[:-1])
    P = z_trunk.numel() // token_z
    a_z = w.shape[0]
    dev = z_trunk.device
    _check_tensor(z_trunk, "pair_cond_f32 z_trunk", F32, lead + (token_z,), dev)
    _check_tensor(rel, "pair_cond_f32 rel", F32, lead + (c_rel,), dev)
    _check_tensor(ln_w, "pair_cond_f32 norm.weight", F32, (token_z + c_rel,), dev)
    _check_tensor(ln_b, "pair_cond_f32 norm.bias", F32, (token_z + c_rel,), dev)
    _check_tensor(w, "pair_cond_f32 proj.weight", F32, (a_z, token_z + c_rel), dev)
    _check_tensor(out, "pair_cond_f32 out", F32, lead + (a_z,), dev)
    need = pair_cond_f32_workspace_bytes(P, token_z, c_rel)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_pair_cond_proj_fwd_f32(
        _ptr(z_trunk), _ptr(rel), _ptr(ln_w), _ptr(ln_b), _ptr(w), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()),
        P, token_z, c_rel, a_z, _stream(z_trunk),
    )
    check(rc, "bioemu_pair_cond_proj_fwd_f32")
    return out


# ----------------------------------------------------------------------------
# Pair glue: distogram head, pairwise-conditioning projection
# ----------------------------------------------------------------------------
def launch_distogram(z: Tensor, w: Tensor, b: Tensor, out: Tensor) -> Tensor:
    require_gpu(z, "distogram")
    if z.ndim != 4 or z.shape[1] != z.shape[2]:
        raise ValueError(f"distogram: z must be [B,N,N,c_z], got {tuple(z.shape)}")
    B, N, _, c_z = z.shape
    nb = w.shape[0]
    dev = z.device
    _check_tensor(z, "distogram z", BF16, (B, N, N, c_z), dev)
    _check_tensor(w, "distogram.weight", BF16, (nb, c_z), dev)
    _check_tensor(b, "distogram.bias", torch.float32, (nb,), dev)
    if out.dtype not in (BF16, torch.float32):
        raise ValueError(f"distogram out: dtype {out.dtype} (bf16 or fp32)")
    _check_tensor(out, "distogram out", out.dtype, (B, N, N, nb), dev)
    rc = lib().bioemu_distogram_fwd(_ptr(z), _ptr(w), _ptr(b), _ptr(out), B, N, c_z, nb,
                                    int(out.dtype == torch.float32), _stream(z))
    check(rc, "bioemu_distogram_fwd")
    return out


def pair_cond_workspace_bytes(token_z: int, c_rel: int, a_z: int) -> int:
    return int(lib().bioemu_pair_cond_workspace_bytes(token_z, c_rel, a_z))


def launch_pair_cond_proj(
    z: Tensor, rel: Tensor, ln_w: Tensor, ln_b: Tensor, w: Tensor, out: Tensor, ws: Tensor | None = None,
    out_tail: Tensor | None = None,
) -> Tensor:
    require_gpu(z, "pairwise_conditioning")
    token_z, c_rel, a_z = z.shape[-1], rel.shape[-1], w.shape[0]
    P = z.numel() // token_z
    dev = z.device
    _check_tensor(z, "pair_cond z_trunk", BF16, tuple(z.shape), dev)
    _check_tensor(rel, "pair_cond rel_pos", BF16, tuple(z.shape[:-1]) + (c_rel,), dev)
    _check_tensor(ln_w, "pair_cond norm.weight", torch.float32, (token_z + c_rel,), dev)
    _check_tensor(ln_b, "pair_cond norm.bias", torch.float32, (token_z + c_rel,), dev)
    _check_tensor(w, "pair_cond proj.weight", BF16, (a_z, token_z + c_rel), dev)
    _check_tensor(out, "pair_cond out", BF16, tuple(z.shape[:-1]) + (a_z,), dev)
    if out_tail is not None:
        _check_tensor(out_tail, "pair_cond out tail", torch.int8, tuple(out.shape), dev)
    need = pair_cond_workspace_bytes(token_z, c_rel, a_z)
    if ws is None or ws.numel() < need:
        ws = workspace(max(need, 1), dev)
    rc = lib().bioemu_pair_cond_proj_fwd(
        _ptr(z), _ptr(rel), _ptr(ln_w), _ptr(ln_b), _ptr(w), _ptr(out), _ptr(out_tail), _ptr(ws),
        ctypes.c_size_t(ws.numel()), P, token_z, c_rel, a_z, _stream(z),
    )
    check(rc, "bioemu_pair_cond_proj_fwd")
    return out


# ----------------------------------------------------------------------------
# Outer product mean
# ----------------------------------------------------------------------------
def opm_workspace_bytes(B: int, S: int, N: int, c_in: int = 64, c_hidden: int = 32) -> int:
    return int(lib().bioemu_opm_workspace_bytes(B, S, N, c_in, c_hidden))


def opm_mask3(mask: Tensor, B: int, S: int, N: int) -> tuple[Tensor, bool]:
    """Reference mask -> ([B,S,N] uint8, mean over rows?).

    A [B,S,N] mask is used as is (divisor = count of rows with any valid
    entry).  A 2-D mask is broadcast exactly as ``masked_fill_(~mask.unsqueeze(-1))``
    broadcasts it against ``[B,S,N,2C]`` (its first dim lines up with S) and
    the divisor is 1 (outer_product_mean.py:62, :69-70).
    """
    if mask.ndim == 3:
        if tuple(mask.shape) != (B, S, N):
            raise ValueError(f"opm: mask shape {tuple(mask.shape)} != {(B, S, N)}")
        return mask_u8(mask), True
    if mask.ndim == 2:
        m3 = torch.broadcast_to(mask.bool(), (S, N)).unsqueeze(0).expand(B, S, N)
        return mask_u8(m3.contiguous()), False
    raise ValueError(f"opm: mask must be [B,S,N] or [B,N], got {tuple(mask.shape)}")


def launch_opm(
    m: Tensor,
    mask3: Tensor,
    mean_rows: bool,
    norm_w: Tensor,
    norm_b: Tensor,
    w_ab: Tensor,
    w_o: Tensor,
    b_o: Tensor,
    out: Tensor,
    z_res: Tensor | None = None,
    ws: Tensor | None = None,
    tail: Tensor | None = None,
) -> Tensor:
    require_gpu(m, "outer_product_mean")
    if m.ndim != 4:
        raise ValueError(f"opm: m must be [B,S,N,C], got {tuple(m.shape)}")
    B, S, N, c_in = m.shape
    c_h = w_ab.shape[0] // 2
    c_out = w_o.shape[0]
    dev = m.device
    _check_tensor(m, "opm m", BF16, (B, S, N, c_in), dev)
    _check_tensor(mask3, "opm mask", torch.uint8, (B, S, N), dev)
    _check_tensor(norm_w, "opm norm.weight", torch.float32, (c_in,), dev)
    _check_tensor(norm_b, "opm norm.bias", torch.float32, (c_in,), dev)
    _check_tensor(w_ab, "opm proj_ab.weight", BF16, (2 * c_h, c_in), dev)
    _check_tensor(w_o, "opm proj_o.weight", BF16, (c_out, c_h * c_h), dev)
    _check_tensor(b_o, "opm proj_o.bias", torch.float32, (c_out,), dev)
    _check_tensor(out, "opm out", BF16, (B, N, N, c_out), dev)
    if z_res is not None:
        _check_tensor(z_res, "opm z", BF16, (B, N, N, c_out), dev)
    _check_tail(tail, out, z_res is not None, "opm")
    need = opm_workspace_bytes(B, S, N, c_in, c_h)
    if need == 0:
        raise ValueError(f"opm: unsupported widths c_in={c_in} c_hidden={c_h}")
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_opm_fwd(
        _ptr(m), _ptr(mask3), int(bool(mean_rows)), _ptr(norm_w), _ptr(norm_b), _ptr(w_ab), _ptr(w_o), _ptr(b_o),
        _ptr(z_res), _ptr(out), _ptr(tail), _ptr(ws), ctypes.c_size_t(ws.numel()), B, S, N, c_in, c_h, c_out,
        _stream(m),
    )
    check(rc, "bioemu_opm_fwd")
    return out


# ----------------------------------------------------------------------------
# Pair-weighted averaging (MSA module)
# ----------------------------------------------------------------------------
def pwa_workspace_bytes(B: int, S: int, N: int, c_m: int, c_h: int, H: int) -> int:
    return int(lib().bioemu_pwa_workspace_bytes(B, S, N, c_m, c_h, H))


def launch_pwa(
    m: Tensor,
    z: Tensor,
    mask_u8: Tensor,
    norm_m_w: Tensor,
    norm_m_b: Tensor,
    w_m: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    out: Tensor,
    num_heads: int,
    residual: bool = False,
    ws: Tensor | None = None,
    tail: Tensor | None = None,
) -> Tensor:
    require_gpu(m, "pair_weighted_averaging")
    if m.ndim != 4 or z.ndim != 4:
        raise ValueError(f"pwa: m must be [B,S,N,c_m] and z [B,N,N,c_z], got {tuple(m.shape)}, {tuple(z.shape)}")
    B, S, N, c_m = m.shape
    c_z = z.shape[-1]
    H = num_heads
    c_h = w_m.shape[0] // H
    dev = m.device
    _check_tensor(m, "pwa m", BF16, (B, S, N, c_m), dev)
    _check_tensor(z, "pwa z", BF16, (B, N, N, c_z), dev)
    _check_tensor(mask_u8, "pwa mask", torch.uint8, (B, N, N), dev)
    _check_tensor(norm_m_w, "pwa norm_m.weight", torch.float32, (c_m,), dev)
    _check_tensor(norm_m_b, "pwa norm_m.bias", torch.float32, (c_m,), dev)
    _check_tensor(w_m, "pwa proj_m.weight", BF16, (H * c_h, c_m), dev)
    _check_tensor(w_g, "pwa proj_g.weight", BF16, (H * c_h, c_m), dev)
    _check_tensor(norm_z_w, "pwa norm_z.weight", torch.float32, (c_z,), dev)
    if norm_z_b is not None:
        _check_tensor(norm_z_b, "pwa norm_z.bias", torch.float32, (c_z,), dev)
    _check_tensor(w_z, "pwa proj_z.weight", BF16, (H, c_z), dev)
    _check_tensor(w_o, "pwa proj_o.weight", BF16, (c_m, H * c_h), dev)
    _check_tensor(out, "pwa out", BF16, (B, S, N, c_m), dev)
    _check_tail(tail, out, residual, "pwa")
    need = pwa_workspace_bytes(B, S, N, c_m, c_h, H)
    if need == 0:
        raise ValueError(f"pwa: unsupported widths c_m={c_m} c_h={c_h} heads={H} (supported: 64, 32, 8)")
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_pwa_fwd(
        _ptr(m), _ptr(z), _ptr(mask_u8), _ptr(norm_m_w), _ptr(norm_m_b), _ptr(w_m), _ptr(w_g), _ptr(norm_z_w),
        _ptr(norm_z_b), _ptr(w_z), _ptr(w_o), _ptr(out), _ptr(tail), _ptr(ws), ctypes.c_size_t(ws.numel()),
        B, S, N, c_m, c_z, c_h, H, int(bool(residual)), _stream(m),
    )
    check(rc, "bioemu_pwa_fwd")
    return out


@torch.library.custom_op("bioemu_mi355x::pair_weighted_averaging", mutates_args=(), device_types="cuda")
def pair_weighted_averaging(
    m: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_m_w: Tensor,
    norm_m_b: Tensor,
    w_m: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    num_heads: int,
) -> Tensor:
    mb = m.to(BF16).contiguous()
    out = torch.empty_like(mb)
    f32 = torch.float32
    launch_pwa(
        mb, z.to(BF16).contiguous(), mask_u8(mask), norm_m_w.to(f32).contiguous(), norm_m_b.to(f32).contiguous(),
        w_m.to(BF16).contiguous(), w_g.to(BF16).contiguous(), norm_z_w.to(f32).contiguous(),
        None if norm_z_b is None else norm_z_b.to(f32).contiguous(), w_z.to(BF16).contiguous(),
        w_o.to(BF16).contiguous(), out, num_heads,
    )
    return out.to(m.dtype)


@pair_weighted_averaging.register_fake
def _(m, z, mask, norm_m_w, norm_m_b, w_m, w_g, norm_z_w, norm_z_b, w_z, w_o, num_heads):
    return torch.empty_like(m)


@torch.library.custom_op("bioemu_mi355x::outer_product_mean", mutates_args=(), device_types="cuda")
def outer_product_mean(
    m: Tensor, mask: Tensor, norm_w: Tensor, norm_b: Tensor, w_ab: Tensor, w_o: Tensor, b_o: Tensor
) -> Tensor:
    mb = m.to(BF16).contiguous()
    B, S, N, _ = mb.shape
    mask3, mean_rows = opm_mask3(mask, B, S, N)
    out = torch.empty(B, N, N, w_o.shape[0], dtype=BF16, device=m.device)
    f32 = torch.float32
    launch_opm(
        mb, mask3, mean_rows, norm_w.to(f32).contiguous(), norm_b.to(f32).contiguous(), w_ab.to(BF16).contiguous(),
        w_o.to(BF16).contiguous(), b_o.to(f32).contiguous(), out,
    )
    return out.to(m.dtype)


@outer_product_mean.register_fake
def _(m, mask, norm_w, norm_b, w_ab, w_o, b_o):
    B, S, N, _ = m.shape
    return m.new_empty(B, N, N, w_o.shape[0])


def opm_f32_workspace_bytes(B: int, S: int, N: int, c_in: int, c_h: int) -> int:
    return int(lib().bioemu_opm_f32_workspace_bytes(B, S, N, c_in, c_h))


def launch_opm_f32(
    m: Tensor,
    mask3: Tensor,
    mean_rows: bool,
    norm_w: Tensor,
    norm_b: Tensor,
    w_ab: Tensor,
    w_o: Tensor,
    b_o: Tensor,
    out: Tensor,
    z_res: Tensor | None = None,
    ws: Tensor | None = None,
) -> Tensor:
    """OuterProductMean in IEEE fp32 (``bioemu_opm_fwd_f32``): every tensor fp32; ``out`` = OPM(m) (+ z_res)."""
    require_gpu(m, "outer_product_mean_f32")
    if m.ndim != 4:
        raise ValueError(f"opm_f32: m must be [B,S,N,C], got {tuple(m.shape)}")
    B, S, N, c_in = m.shape
    c_h = w_ab.shape[0] // 2
    c_out = w_o.shape[0]
    dev = m.device
    _check_tensor(m, "opm_f32 m", F32, (B, S, N, c_in), dev)
    _check_tensor(mask3, "opm_f32 mask", torch.uint8, (B, S, N), dev)
    for name, t, shp in (
        ("norm.weight", norm_w, (c_in,)), ("norm.bias", norm_b, (c_in,)), ("proj_ab.weight", w_ab, (2 * c_h, c_in)),
        ("proj_o.weight", w_o, (c_out, c_h * c_h)), ("proj_o.bias", b_o, (c_out,)),
    ):
        _check_tensor(t, f"opm_f32 {name}", F32, shp, dev)
    _check_tensor(out, "opm_f32 out", F32, (B, N, N, c_out), dev)
    if z_res is not None:
        _check_tensor(z_res, "opm_f32 z_res", F32, (B, N, N, c_out), dev)
    need = opm_f32_workspace_bytes(B, S, N, c_in, c_h)
    if need == 0:
        raise ValueError(f"opm_f32: unsupported widths c_in={c_in} c_hidden={c_h} (c_hidden must be 32)")
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_opm_fwd_f32(
        _ptr(m), _ptr(mask3), int(bool(mean_rows)), _ptr(norm_w), _ptr(norm_b), _ptr(w_ab), _ptr(w_o), _ptr(b_o),
        _ptr(z_res), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()), B, S, N, c_in, c_h, c_out, _stream(m),
    )
    check(rc, "bioemu_opm_fwd_f32")
    return out


@torch.library.custom_op("bioemu_mi355x::outer_product_mean_f32", mutates_args=(), device_types="cuda")
def outer_product_mean_f32(
    m: Tensor, mask: Tensor, norm_w: Tensor, norm_b: Tensor, w_ab: Tensor, w_o: Tensor, b_o: Tensor
) -> Tensor:
    mf = m.to(F32).contiguous()
    B, S, N, _ = mf.shape
    mask3, mean_rows = opm_mask3(mask, B, S, N)
    out = torch.empty(B, N, N, w_o.shape[0], dtype=F32, device=m.device)
    f32c = lambda t: t.to(F32).contiguous()  # noqa: E731
    launch_opm_f32(mf, mask3, mean_rows, f32c(norm_w), f32c(norm_b), f32c(w_ab), f32c(w_o), f32c(b_o), out)
    return out


@outer_product_mean_f32.register_fake
def _(m, mask, norm_w, norm_b, w_ab, w_o, b_o):
    B, S, N, _ = m.shape
    return m.new_empty(B, N, N, w_o.shape[0], dtype=F32)


def pwa_f32_workspace_bytes(B: int, S: int, N: int, c_m: int, c_h: int, H: int) -> int:
    return int(lib().bioemu_pwa_f32_workspace_bytes(B, S, N, c_m, c_h, H))


def launch_pwa_f32(
    m: Tensor,
    z: Tensor,
    mask_u8: Tensor,
    norm_m_w: Tensor,
    norm_m_b: Tensor,
    w_m: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    out: Tensor,
    num_heads: int,
    residual: bool = False,
    inf: float = 1e6,
    ws: Tensor | None = None,
) -> Tensor:
    """PairWeightedAveraging in IEEE fp32 (``bioemu_pwa_fwd_f32``): every tensor fp32; ``out`` = PWA(m, z)
    (+ m with ``residual``; ``out`` may be ``m`` then)."""
    require_gpu(m, "pair_weighted_averaging_f32")
    if m.ndim != 4 or z.ndim != 4:
        raise ValueError(f"pwa_f32: m must be [B,S,N,c_m] and z [B,N,N,c_z], got {tuple(m.shape)}, {tuple(z.shape)}")
    B, S, N, c_m = m.shape
    c_z = z.shape[-1]
    H = num_heads
    c_h = w_m.shape[0] // H
    dev = m.device
    _check_tensor(m, "pwa_f32 m", F32, (B, S, N, c_m), dev)
    _check_tensor(z, "pwa_f32 z", F32, (B, N, N, c_z), dev)
    _check_tensor(mask_u8, "pwa_f32 mask", torch.uint8, (B, N, N), dev)
    for name, t, shp in (
        ("norm_m.weight", norm_m_w, (c_m,)), ("norm_m.bias", norm_m_b, (c_m,)), ("proj_m.weight", w_m, (H * c_h, c_m)),
        ("proj_g.weight", w_g, (H * c_h, c_m)), ("norm_z.weight", norm_z_w, (c_z,)), ("proj_z.weight", w_z, (H, c_z)),
        ("proj_o.weight", w_o, (c_m, H * c_h)),
    ):
        _check_tensor(t, f"pwa_f32 {name}", F32, shp, dev)
    if norm_z_b is not None:
        _check_tensor(norm_z_b, "pwa_f32 norm_z.bias", F32, (c_z,), dev)
    _check_tensor(out, "pwa_f32 out", F32, (B, S, N, c_m), dev)
    need = pwa_f32_workspace_bytes(B, S, N, c_m, c_h, H)
    if need == 0:
        raise ValueError(f"pwa_f32: unsupported widths c_m={c_m} c_h={c_h} heads={H} (c_h must be 32)")
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_pwa_fwd_f32(
        _ptr(m), _ptr(z), _ptr(mask_u8), _ptr(norm_m_w), _ptr(norm_m_b), _ptr(norm_z_w), _ptr(norm_z_b), _ptr(w_m),
        _ptr(w_g), _ptr(w_z), _ptr(w_o), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()), B, S, N, c_m, c_z, c_h, H,
        float(inf), int(bool(residual)), _stream(m),
    )
    check(rc, "bioemu_pwa_fwd_f32")
    return out


@torch.library.custom_op("bioemu_mi355x::pair_weighted_averaging_f32", mutates_args=(), device_types="cuda")
def pair_weighted_averaging_f32(
    m: Tensor,
    z: Tensor,
    mask: Tensor,
    norm_m_w: Tensor,
    norm_m_b: Tensor,
    w_m: Tensor,
    w_g: Tensor,
    norm_z_w: Tensor,
    norm_z_b: Tensor | None,
    w_z: Tensor,
    w_o: Tensor,
    num_heads: int,
    inf: float,
) -> Tensor:
    mf = m.to(F32).contiguous()
    out = torch.empty_like(mf)
    f32c = lambda t: None if t is None else t.to(F32).contiguous()  # noqa: E731
    launch_pwa_f32(mf, f32c(z), mask_u8(mask), f32c(norm_m_w), f32c(norm_m_b), f32c(w_m), f32c(w_g), f32c(norm_z_w),
                   f32c(norm_z_b), f32c(w_z), f32c(w_o), out, num_heads, inf=inf)
    return out


@pair_weighted_averaging_f32.register_fake
def _(m, z, mask, norm_m_w, norm_m_b, w_m, w_g, norm_z_w, norm_z_b, w_z, w_o, num_heads, inf):
    return m.new_empty(m.shape, dtype=F32)


# ----------------------------------------------------------------------------
# PairMixer trunk glue: recycling updates and the MSA input embedding
# ----------------------------------------------------------------------------
def launch_ln_linear(
    x: Tensor,
    norm_w: Tensor,
    norm_b: Tensor,
    w: Tensor,
    base: Tensor,
    out: Tensor,
    base_tail: Tensor | None = None,
    out_tail: Tensor | None = None,
    ws: Tensor | None = None,
) -> Tensor:
    """``out = base + w LN(x)`` over rows (the recycling update, pairmixer.py:281-282): pair rows of 128
    channels (4-d x) through the pair kernel, token rows (3-d x) through the token LayerNorm + GEMM."""
    require_gpu(x, "ln_linear")
    D = x.shape[-1]
    M = x.numel() // D
    dev = x.device
    for t, what in ((x, "x"), (base, "base"), (out, "out")):
        _check_tensor(t, f"ln_linear {what}", BF16, tuple(x.shape), dev)
    _check_tensor(w, "ln_linear weight", BF16, (D, D), dev)
    _check_tensor(norm_w, "ln_linear norm.weight", torch.float32, (D,), dev)
    _check_tensor(norm_b, "ln_linear norm.bias", torch.float32, (D,), dev)
    for t, what in ((base_tail, "base tail"), (out_tail, "out tail")):
        if t is not None:
            _check_tensor(t, f"ln_linear {what}", torch.int8, tuple(x.shape), dev)
    pair = x.dim() == 4
    need = (lib().bioemu_pair_ln_linear_workspace_bytes(D) if pair
            else lib().bioemu_token_ln_linear_workspace_bytes(M, D))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    fn = lib().bioemu_pair_ln_linear_fwd if pair else lib().bioemu_token_ln_linear_fwd
    rc = fn(_ptr(x), _ptr(norm_w), _ptr(norm_b), _ptr(w), _ptr(base), _ptr(base_tail), _ptr(out), _ptr(out_tail),
            _ptr(ws), ctypes.c_size_t(ws.numel()), M, D, _stream(x))
    check(rc, "bioemu_pair_ln_linear_fwd" if pair else "bioemu_token_ln_linear_fwd")
    return out


def launch_ln_linear_f32(
    x: Tensor, norm_w: Tensor, norm_b: Tensor, w: Tensor, base: Tensor | None, out: Tensor, ws: Tensor | None = None
) -> Tensor:
    """``out = (base +) w LN(x)`` over rows in IEEE fp32 (``bioemu_ln_linear_fwd_f32``; the recycling updates of
    a trunk run with autocast off, pairmixer.py:281-282)."""
    require_gpu(x, "ln_linear_f32")
    K = x.shape[-1]
    N = w.shape[0]
    M = x.numel() // K
    dev = x.device
    _check_tensor(x, "ln_linear_f32 x", F32, tuple(x.shape), dev)
    _check_tensor(w, "ln_linear_f32 weight", F32, (N, K), dev)
    _check_tensor(norm_w, "ln_linear_f32 norm.weight", F32, (K,), dev)
    _check_tensor(norm_b, "ln_linear_f32 norm.bias", F32, (K,), dev)
    oshape = tuple(x.shape[:-1]) + (N,)
    _check_tensor(out, "ln_linear_f32 out", F32, oshape, dev)
    if base is not None:
        _check_tensor(base, "ln_linear_f32 base", F32, oshape, dev)
    need = int(lib().bioemu_ln_linear_f32_workspace_bytes(M, K))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_ln_linear_fwd_f32(_ptr(x), _ptr(norm_w), _ptr(norm_b), _ptr(w), _ptr(base), _ptr(out),
                                        _ptr(ws), ctypes.c_size_t(ws.numel()), M, K, N, _stream(x))
    check(rc, "bioemu_ln_linear_fwd_f32")
    return out


def trunk_uncond_f32_workspace_bytes(P: int, D: int, hidden: int) -> int:
    return int(lib().bioemu_trunk_uncond_f32_workspace_bytes(P, D, hidden))


def launch_trunk_uncond_f32(
    z_init: Tensor, z_norm_w: Tensor, z_norm_b: Tensor, t_norm_w: Tensor, t_norm_b: Tensor, fc1_w: Tensor,
    fc2_w: Tensor, fc3_w: Tensor, out: Tensor, ws: Tensor | None = None,
) -> Tensor:
    """``out = z_init + uncond_transition(z_norm(z_init))`` in IEEE fp32 (pairmixer.py:266-273)."""
    require_gpu(z_init, "trunk_uncond_f32")
    D = z_init.shape[-1]
    P = z_init.numel() // D
    hidden = fc1_w.shape[0]
    dev = z_init.device
    _check_tensor(z_init, "trunk_uncond_f32 z_init", F32, tuple(z_init.shape), dev)
    _check_tensor(out, "trunk_uncond_f32 out", F32, tuple(z_init.shape), dev)
    for name, t, shp in (
        ("z_norm.weight", z_norm_w, (D,)), ("z_norm.bias", z_norm_b, (D,)), ("norm.weight", t_norm_w, (D,)),
        ("norm.bias", t_norm_b, (D,)), ("fc1.weight", fc1_w, (hidden, D)), ("fc2.weight", fc2_w, (hidden, D)),
        ("fc3.weight", fc3_w, (D, hidden)),
    ):
        _check_tensor(t, f"trunk_uncond_f32 {name}", F32, shp, dev)
    need = trunk_uncond_f32_workspace_bytes(P, D, hidden)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_trunk_uncond_fwd_f32(
        _ptr(z_init), _ptr(z_norm_w), _ptr(z_norm_b), _ptr(t_norm_w), _ptr(t_norm_b), _ptr(fc1_w), _ptr(fc2_w),
        _ptr(fc3_w), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()), P, D, hidden, _stream(z_init))
    check(rc, "bioemu_trunk_uncond_fwd_f32")
    return out


def launch_distogram_f32(z: Tensor, w: Tensor, b: Tensor, out: Tensor, ws: Tensor | None = None) -> Tensor:
    """``out = (z + z^T) w^T + b`` in IEEE fp32 (embedders.py:191-206)."""
    require_gpu(z, "distogram_f32")
    if z.ndim != 4 or z.shape[1] != z.shape[2]:
        raise ValueError(f"distogram_f32: z must be [B,N,N,c_z], got {tuple(z.shape)}")
    B, N, _, c_z = z.shape
    nb = w.shape[0]
    dev = z.device
    _check_tensor(z, "distogram_f32 z", F32, (B, N, N, c_z), dev)
    _check_tensor(w, "distogram_f32 weight", F32, (nb, c_z), dev)
    _check_tensor(b, "distogram_f32 bias", F32, (nb,), dev)
    _check_tensor(out, "distogram_f32 out", F32, (B, N, N, nb), dev)
    need = int(lib().bioemu_distogram_f32_workspace_bytes(B, N, c_z))
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_distogram_fwd_f32(_ptr(z), _ptr(w), _ptr(b), _ptr(out), _ptr(ws), ctypes.c_size_t(ws.numel()),
                                        B, N, c_z, nb, _stream(z))
    check(rc, "bioemu_distogram_fwd_f32")
    return out


def launch_msa_embed_f32(
    msa: Tensor, has_deletion: Tensor, deletion_value: Tensor, msa_paired: Tensor | None, emb: Tensor,
    w_msa: Tensor, w_s: Tensor, m: Tensor, ws: Tensor | None = None,
) -> Tensor:
    """MSA input embedding (pairmixer.py:591-599) into an fp32 ``m`` (a trunk run with autocast off)."""
    require_gpu(msa, "msa_embed_f32")
    B, R, T, F0 = msa.shape
    E = emb.shape[-1]
    C = w_msa.shape[0]
    dev = msa.device
    _check_tensor(msa, "msa_embed_f32 msa", F32, (B, R, T, F0), dev)
    for t, what in ((has_deletion, "has_deletion"), (deletion_value, "deletion_value"), (msa_paired, "msa_paired")):
        if t is not None:
            _check_tensor(t, f"msa_embed_f32 {what}", F32, (B, R, T), dev)
    _check_tensor(emb, "msa_embed_f32 emb", F32, (B, T, E), dev)
    _check_tensor(w_msa, "msa_embed_f32 msa_proj.weight", F32, (C, F0 + 2 + int(msa_paired is not None)), dev)
    _check_tensor(w_s, "msa_embed_f32 s_proj.weight", F32, (C, E), dev)
    _check_tensor(m, "msa_embed_f32 m", F32, (B, R, T, C), dev)
    need = lib().bioemu_msa_embed_workspace_bytes(B, T)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_msa_embed_fwd_f32(
        _ptr(msa), _ptr(has_deletion), _ptr(deletion_value), _ptr(msa_paired), _ptr(emb), _ptr(w_msa), _ptr(w_s),
        _ptr(m), _ptr(ws), ctypes.c_size_t(ws.numel()), B, R, T, F0, E, C, _stream(msa),
    )
    check(rc, "bioemu_msa_embed_fwd_f32")
    return m


def trunk_uncond_workspace_bytes(P: int, D: int, hidden: int) -> int:
    return int(lib().bioemu_trunk_uncond_workspace_bytes(P, D, hidden))


def launch_trunk_uncond(
    z_init: Tensor,
    z_norm_w: Tensor,
    z_norm_b: Tensor,
    t_norm_w: Tensor,
    t_norm_b: Tensor,
    fc1_w: Tensor,
    fc2_w: Tensor,
    fc3_w: Tensor,
    out: Tensor,
    z_init_tail: Tensor | None = None,
    out_tail: Tensor | None = None,
    ws: Tensor | None = None,
) -> Tensor:
    """``out = z_init + uncond_transition(z_norm(z_init))`` over pair rows of 128 channels (the unconditional
    branch, pairmixer.py:266-273); the tails carry z_init and out as residual streams (both or neither)."""
    require_gpu(z_init, "trunk_uncond")
    D = z_init.shape[-1]
    P = z_init.numel() // D
    dev = z_init.device
    hidden = fc1_w.shape[0]
    _check_tensor(z_init, "trunk_uncond z_init", BF16, tuple(z_init.shape), dev)
    _check_tensor(out, "trunk_uncond out", BF16, tuple(z_init.shape), dev)
    for t, what in ((z_norm_w, "z_norm.weight"), (z_norm_b, "z_norm.bias"), (t_norm_w, "norm.weight"),
                    (t_norm_b, "norm.bias")):
        _check_tensor(t, f"trunk_uncond {what}", torch.float32, (D,), dev)
    _check_tensor(fc1_w, "trunk_uncond fc1.weight", BF16, (hidden, D), dev)
    _check_tensor(fc2_w, "trunk_uncond fc2.weight", BF16, (hidden, D), dev)
    _check_tensor(fc3_w, "trunk_uncond fc3.weight", BF16, (D, hidden), dev)
    if (z_init_tail is None) != (out_tail is None):
        raise ValueError("trunk_uncond: z_init_tail and out_tail go together")
    for t, what in ((z_init_tail, "z_init tail"), (out_tail, "out tail")):
        if t is not None:
            _check_tensor(t, f"trunk_uncond {what}", torch.int8, tuple(z_init.shape), dev)
    need = trunk_uncond_workspace_bytes(P, D, hidden)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_trunk_uncond_fwd(
        _ptr(z_init), _ptr(z_init_tail), _ptr(z_norm_w), _ptr(z_norm_b), _ptr(t_norm_w), _ptr(t_norm_b), _ptr(fc1_w),
        _ptr(fc2_w), _ptr(fc3_w), _ptr(out), _ptr(out_tail), _ptr(ws), ctypes.c_size_t(ws.numel()), P, D, hidden,
        _stream(z_init),
    )
    check(rc, "bioemu_trunk_uncond_fwd")
    return out


def launch_msa_embed(
    msa: Tensor,
    has_deletion: Tensor,
    deletion_value: Tensor,
    msa_paired: Tensor | None,
    emb: Tensor,
    w_msa: Tensor,
    w_s: Tensor,
    m: Tensor,
    m_tail: Tensor,
    ws: Tensor | None = None,
) -> Tensor:
    """MSA input embedding (pairmixer.py:591-599) into the MSA stream ``m`` (bf16) and its int8 tail."""
    require_gpu(msa, "msa_embed")
    B, R, T, F0 = msa.shape
    E = emb.shape[-1]
    C = w_msa.shape[0]
    dev = msa.device
    f32 = torch.float32
    _check_tensor(msa, "msa_embed msa", f32, (B, R, T, F0), dev)
    for t, what in ((has_deletion, "has_deletion"), (deletion_value, "deletion_value"), (msa_paired, "msa_paired")):
        if t is not None:
            _check_tensor(t, f"msa_embed {what}", f32, (B, R, T), dev)
    _check_tensor(emb, "msa_embed emb", f32, (B, T, E), dev)
    _check_tensor(w_msa, "msa_embed msa_proj.weight", f32, (C, F0 + 2 + int(msa_paired is not None)), dev)
    _check_tensor(w_s, "msa_embed s_proj.weight", f32, (C, E), dev)
    _check_tensor(m, "msa_embed m", BF16, (B, R, T, C), dev)
    _check_tensor(m_tail, "msa_embed m tail", torch.int8, (B, R, T, C), dev)
    need = lib().bioemu_msa_embed_workspace_bytes(B, T)
    if ws is None or ws.numel() < need:
        ws = workspace(need, dev)
    rc = lib().bioemu_msa_embed_fwd(
        _ptr(msa), _ptr(has_deletion), _ptr(deletion_value), _ptr(msa_paired), _ptr(emb), _ptr(w_msa), _ptr(w_s),
        _ptr(m), _ptr(m_tail), _ptr(ws), ctypes.c_size_t(ws.numel()), B, R, T, F0, E, C, _stream(msa),
    )
    check(rc, "bioemu_msa_embed_fwd")
    return m
