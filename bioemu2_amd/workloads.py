"""Synthetic, HBM-resident workloads for the benchmark configs.

Each workload owns its seeded inputs, random-init weights, preallocated
outputs, workspaces and masks, so ``step()`` launches kernels and allocates
nothing (except the out-of-place ones: config 1 and the PairMixer trunk pass
build their fp32 <-> bf16 + tail streams and masks through torch's caching
allocator, as a caller of ``forward`` would).
``kernel_work(name)`` gives the algorithmic work of one launch of a named
kernel at the workload's shape: ``("mfma", flops)`` or ``("hbm", bytes)``,
chosen by comparing the kernel's flops per minimum HBM byte with the MI355X
ridge point (2.5 PFLOP/s / 8 TB/s ~ 312 flop/B).
"""

from __future__ import annotations

import json
import math
import time
from pathlib import Path

import torch
from torch import Tensor

from . import _ops

RIDGE = 2500e12 / 8000e9
_PROFILES = Path(__file__).resolve().parents[1] / "profiles" / "traffic.json"


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters, if recorded on the current kernel sources
    (None when absent or measured on other sources)."""
    from .profiling import csrc_hash

    try:
        entry = json.loads(_PROFILES.read_text()).get(workload, {})
    except (OSError, ValueError):
        return None
    if entry.get("csrc_sha16") != csrc_hash():
        return None
    return entry.get("kernels", {}).get(kernel)


def token_mask(n: int, n_pad: int, device, batch: int = 1) -> Tensor:
    """Valid tokens first, the last ``n_pad`` padded (deterministic trailing padding)."""
    m = torch.ones(batch, n, dtype=torch.bool)
    if n_pad:
        m[:, n - n_pad:] = False
    return m.to(device)


def init_module(module: torch.nn.Module, seed: int = 0) -> torch.nn.Module:
    """Module default init under ``manual_seed(seed)``, then zero params re-drawn N(0, 0.02)."""
    with torch.no_grad():
        g = torch.Generator().manual_seed(seed + 1)
        for p in module.parameters():
            if torch.count_nonzero(p) == 0:
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    return module


def _bound(flops: float, nbytes: float) -> tuple[str, float]:
    if nbytes <= 0 or flops / nbytes > RIDGE:
        return ("mfma", float(flops))
    return ("hbm", float(nbytes))


# ----------------------------------------------------------------------------
# Per-kernel algorithmic work.  P = B*N*N pairs, c = 128 channels, bf16 = 2 B.
# ----------------------------------------------------------------------------
def trimul_kernel_work(name: str, B: int, N: int, c: int = 128) -> tuple[str, float] | None:
    P = B * N * N
    if name == "trimul_proj_in":
        # LN + [p_in | g_in] (c -> 4c) ; reads x, writes a and b planes
        return ("hbm", float(P * (c * 2 + 2 * c * 2)))
    if name == "bgemm_nt":
        # o[d,i,j] = sum_k a[d,i,k] b[d,j,k] over the valid N: the contraction, reported on MFMA
        return ("mfma", 2.0 * B * c * N * N * N)
    if name == "trimul_out":
        # LN_out(o) -> p_out, LN_in(x) -> g_out ; reads o and x, writes out
        return ("hbm", float(3 * P * c * 2))
    if name == "trimul_fold":
        # folds the LayerNorm affines into the output weights: reads 2 c x c bf16, writes them back
        return ("hbm", float(4 * c * c * 2))
    return None


def fold_kernel_work(name: str, launches: int, rows128: int, rows64: int = 0,
                     rows256: int = 0) -> tuple[str, float] | None:
    """LayerNorm folds: W diag(gamma) and W beta, reading and writing each weight once; the amount
    per launch averaged over the step's `launches` folds of `rows128` rows of width 128, `rows64`
    of width 64 and `rows256` of width 256."""
    if name == "fold_ln":
        return ("hbm", float(2 * (rows128 * 128 + rows64 * 64 + rows256 * 256) * 2) / launches)
    return None


def triatt_kernel_work(name: str, B: int, N: int, c: int = 128, H: int = 4,
                       n_valid: int | None = None) -> tuple[str, float] | None:
    """``n_valid``: valid (unpadded) tokens; the attention counts only frame rows with a valid key and, in
    them, the valid keys (a masked key adds an exact zero and the kernel skips whole blocks of them; a row
    without valid keys is the closed-form mean of v), for every query."""
    P = B * N * N
    nv = N if n_valid is None else n_valid
    if name == "triatt_proj":
        # LN + the key side, k, v (c -> 2c) + bias (c -> H): reads z, writes k, v, the bias and the frame mask
        return ("hbm", float(P * (c * 2 + 2 * c * 2 + H * 2 + 1)))
    if name == "triatt_frag":
        # the q and g rows of the projection and Wo ([c][c] each) read and written in fragment order
        return ("hbm", float(2 * 3 * c * c * 2))
    if name == "triatt_flash":
        # q (c -> c) for the queries of rows with a valid key; QK^T and PV over the valid keys for every
        # (valid row, query, head); the gate g (c -> c) and the output projection for every pair
        return ("mfma", 2.0 * B * nv * N * nv * c * 2 + 2.0 * B * nv * N * c * c + 2 * 2.0 * P * c * c)
    return None


class Workload:
    name: str
    metric: str
    config: dict
    flops: float
    dtype: str = "bf16"   # the arithmetic the timed kernels compute in

    def step(self) -> None:
        raise NotImplementedError

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        raise NotImplementedError

    def cpu_sample(self, oracle):
        raise NotImplementedError


class TriMulWorkload(Workload):
    """Config 4: one triangle multiplication (outgoing or incoming) at N=768, bf16."""

    def __init__(self, device, mode: str, n: int = 768, seed: int = 0):
        from .triangle_multiplication import TriangleMultiplicationHip

        self.mode = mode
        self.n = n
        self.n_pad = n // 10
        self.name = f"trimul_{'out' if mode == 'outgoing' else 'in'}_n{n}"
        self.metric = f"ms per triangle multiplication ({mode}) at N={n} bf16"
        self.config = {"workload": self.name, "N": n, "c_z": 128, "batch": 1, "padded_tokens": self.n_pad}
        torch.manual_seed(seed)
        self.module = init_module(TriangleMultiplicationHip(dim=128, mode=mode), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.x_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.x = self.x_cpu.to(device)
        self.tok = token_mask(n, self.n_pad, device)
        self.pair_mask = _ops.mask_u8(self.tok[:, :, None] & self.tok[:, None, :])
        self.out = torch.empty_like(self.x)
        self.ws = _ops.workspace(_ops.trimul_workspace_bytes(1, n, 128), device)
        self.params = self.module.prepared_params()
        self.flops = 2.0 * n * n * 128 * (4 * 128 + 2 * 128) + 2.0 * 128 * n ** 3

    def step(self) -> None:
        _ops.launch_trimul(self.x, self.pair_mask, *self.params, self.out, self.mode == "outgoing", ws=self.ws)

    def cpu_sample(self, oracle):
        """(callable, fraction of one step it computes, description) for the CPU baseline."""
        x = self.x_cpu.float()
        pm = (self.tok[:, :, None] & self.tok[:, None, :]).cpu()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}
        return (lambda: oracle.trimul(x, pm, params, self.mode)), 1.0, f"oracle.trimul fp32, full N={self.n}"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        w = trimul_kernel_work(kernel, 1, self.n)
        if w is None:
            raise KeyError(kernel)
        return w


class TriAttWorkload(Workload):
    """Config 4: one triangle attention (starting or ending node) at N=768, bf16."""

    def __init__(self, device, starting: bool, n: int = 768, seed: int = 0):
        from .triangle_attention import TriangleAttentionHip

        self.starting = starting
        self.n = n
        self.n_pad = n // 10
        node = "start" if starting else "end"
        self.name = f"triatt_{node}_n{n}"
        self.metric = f"ms per triangle attention ({node}ing node) at N={n} bf16"
        self.config = {"workload": self.name, "N": n, "c_z": 128, "heads": 4, "head_dim": 32,
                       "batch": 1, "padded_tokens": self.n_pad}
        torch.manual_seed(seed)
        self.module = init_module(TriangleAttentionHip(128, 4, starting=starting), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.x_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.x = self.x_cpu.to(device)
        self.tok = token_mask(n, self.n_pad, device)
        self.pair_mask = _ops.mask_u8(self.tok[:, :, None] & self.tok[:, None, :])
        self.out = torch.empty_like(self.x)
        self.ws = _ops.workspace(_ops.triatt_workspace_bytes(1, n), device)
        self.params = self.module.prepared_params()
        nv = n - self.n_pad
        self.flops = 2.0 * n * n * 128 * (4 * 128 + 4 + 128) + 2.0 * 2 * nv * n * nv * 128

    def step(self) -> None:
        _ops.launch_triatt(self.x, self.pair_mask, *self.params, self.out, self.starting, ws=self.ws)

    def cpu_sample(self, oracle):
        x = self.x_cpu.float()
        pm = (self.tok[:, :, None] & self.tok[:, None, :]).cpu()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}
        fn = lambda: oracle.triangle_attention(x, pm, params, 4, self.starting, row_chunk=64)  # noqa: E731
        return fn, 1.0, f"oracle.triangle_attention fp32, full N={self.n} (64-row chunks)"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        w = (triatt_kernel_work(kernel, 1, self.n, n_valid=self.n - self.n_pad)
             or fold_kernel_work(kernel, 1, 4 * 128 + 4))
        if w is None:
            raise KeyError(kernel)
        return w


def block_flops(n: int, c: int = 128, cs: int = 384, n_valid: int | None = None) -> float:
    """Algorithmic flops of one Pairformer block at N = n (B = 1).  With ``n_valid`` valid tokens the
    triangle attentions count their valid keys in valid rows only (masked keys add exact zeros), as the
    OPM counts its valid MSA rows; every other term is dense (1361.3 GF at N = 768 when all are valid)."""
    P = n * n
    nv = n if n_valid is None else n_valid
    trimul = 2.0 * P * c * 6 * c + 2.0 * c * n ** 3
    triatt = 2.0 * P * c * (5 * c + 4) + 4.0 * nv * n * nv * c
    trans_z = 2.0 * P * c * 12 * c
    apb = 2.0 * P * c * 16 + 2.0 * n * cs * 5 * cs + 4.0 * n * n * cs
    trans_s = 2.0 * n * cs * 12 * cs
    return 2 * trimul + 2 * triatt + trans_z + apb + trans_s


class BlockWorkload(Workload):
    """The BASELINE metric: one full bf16 Pairformer block at N=768 (config 4 + s [1,768,384]).

    With ``tails`` (the default) the residual streams z and s carry int8 tails, the path held to the
    north_star bound against the fp32 oracle; without them they are plain bf16 (rounded after every add,
    as the reference's bf16-autocast trunk stores them)."""

    cpu_warmup = 1
    cpu_calls = 3

    def __init__(self, device, n: int = 768, seed: int = 0, tails: bool = True):
        from .pairformer import PairformerBlockHip, pair_masks

        self.n = n
        self.tails = tails
        # padded (masked) trailing tokens: 10 % at the BASELINE size (config 4,
        # 76 of 768), 5 % at the 48-block trunk size (config 5, 102 of 2048)
        self.n_pad = n // 20 if n >= 2048 else n // 10
        self.name = f"pairformer_block_n{n}" + ("" if tails else "_bf16stream")
        self.metric = f"ms per Pairformer block at N={n} bf16"
        self.config = {"workload": self.name, "N": n, "c_z": 128, "c_s": 384, "batch": 1,
                       "triatt_heads": 4, "apb_heads": 16, "padded_tokens": self.n_pad,
                       "residual_stream": "bf16 + int8 tail" if tails else "bf16"}
        torch.manual_seed(seed)
        self.module = init_module(PairformerBlockHip(), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.s_cpu = torch.randn(1, n, 384, generator=g).to(torch.bfloat16)
        self.z = self.z_cpu.to(device)
        self.s = self.s_cpu.to(device)
        self.z_tail = torch.zeros(self.z.shape, dtype=torch.int8, device=device) if tails else None
        self.s_tail = torch.zeros(self.s.shape, dtype=torch.int8, device=device) if tails else None
        self.tok = token_mask(n, self.n_pad, device)
        self.masks = pair_masks(self.tok)
        self.ws = _ops.workspace(self.module.workspace_bytes(1, n), device)
        self.flops = block_flops(n, n_valid=n - self.n_pad)

    def step(self) -> None:
        self.module.forward_(self.s, self.z, self.tok, self.s_tail, self.z_tail, ws=self.ws, masks=self.masks)

    def cpu_sample(self, oracle):
        s = self.s_cpu.float()
        z = self.z_cpu.float()
        tok = self.tok.cpu()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}
        fn = lambda: oracle.pairformer_block(s, z, tok, params, triatt_row_chunk=64)  # noqa: E731
        return fn, 1.0, f"oracle.pairformer_block fp32, full N={self.n}"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        n, c, cs = self.n, 128, 384
        w = trimul_kernel_work(kernel, 1, n) or triatt_kernel_work(kernel, 1, n, n_valid=n - self.n_pad)
        if w is not None:
            return w
        if kernel == "fold_ln":  # triatt (516 rows) x2, APB bias (16 rows), transition fc1 + fc2 (1024 rows, one launch)
            return fold_kernel_work(kernel, 4, 2 * 516 + 16 + 1024)
        if kernel == "transition_pair":
            return ("mfma", 2.0 * n * n * c * 12 * c)
        if kernel == "apb_pair_bias":
            return ("hbm", float(n * n * (c * 2 + 16 * 2)))
        if kernel == "apb_flash":
            return ("mfma", 4.0 * n * n * cs)
        # token-side kernels: tiny; report against HBM with their operand bytes
        token_bytes = {
            "token_layernorm": 2 * n * cs * 2,
            "apb_proj_qkvg": n * cs * 2 * 5 + 4 * cs * cs * 2,
            "apb_proj_o": n * cs * 2 * 3 + cs * cs * 2,
            "transition_token_swiglu": n * cs * 2 + n * 4 * cs * 2 + 2 * 4 * cs * cs * 2,
            "transition_token_out": n * 4 * cs * 2 + 2 * n * cs * 2 + 4 * cs * cs * 2,
        }
        if kernel in token_bytes:
            return ("hbm", float(token_bytes[kernel]))
        raise KeyError(kernel)


class Config1Workload(BlockWorkload):
    """Config 1: the reference's CPU-runnable case, one block at N=64 with fp32 z [1,64,64,128] and
    s [1,64,384], all tokens valid.  A step is the out-of-place ``forward`` under bf16 autocast (the trunk's
    policy; the block has no fp32 arithmetic): fp32 in, streams split into bf16 + tail, the block, fp32 out.
    The CPU baseline is the whole fp32 oracle block at the same size."""

    def __init__(self, device, n: int = 64, seed: int = 0):
        super().__init__(device, n, seed)
        self.n_pad = 0
        self.flops = block_flops(n)
        from .pairformer import pair_masks

        self.tok = token_mask(n, 0, device)
        self.masks = pair_masks(self.tok)
        self.name = f"pairformer_block_n{n}_fp32io"
        self.metric = f"ms per Pairformer block at N={n}, fp32 in/out"
        self.config = dict(self.config, workload=self.name, padded_tokens=0, io="fp32")
        self.s32 = self.s_cpu.float().to(device)
        self.z32 = self.z_cpu.float().to(device)

    def step(self) -> None:
        with torch.autocast("cuda", dtype=torch.bfloat16):
            self.module(self.s32, self.z32, self.tok)


class TrunkWorkload(BlockWorkload):
    """Config 5: the full 48-block Pairformer trunk at N=2048 on one GPU (z [1,2048,2048,128] bf16 with its
    int8 tail, s [1,2048,384], 5 % padded tokens), every block's weights random-init, the pair tensor and
    one shared workspace resident in HBM.  A step is one pass through the 48 blocks."""

    cpu_warmup = 0
    cpu_calls = 1

    def __init__(self, device, n: int = 2048, blocks: int = 48, seed: int = 0):
        from .pairformer import PairformerBlockHip

        super().__init__(device, n, seed)
        self.blocks = [self.module] + [init_module(PairformerBlockHip(), seed + 1 + k).to(device).eval()
                                       for k in range(blocks - 1)]
        self.name = f"pairformer_trunk{blocks}_n{n}"
        self.metric = f"ms per {blocks}-block Pairformer trunk pass at N={n} bf16"
        self.config = dict(self.config, workload=self.name, blocks=blocks)
        self.flops = blocks * block_flops(n, n_valid=n - self.n_pad)

    def step(self) -> None:
        for blk in self.blocks:
            blk.forward_(self.s, self.z, self.tok, self.s_tail, self.z_tail, ws=self.ws, masks=self.masks)

    def cpu_sample(self, oracle):
        """One fp32 oracle block at N=512 (5 % padded), scaled to the trunk by algorithmic flops
        (48 x block_flops(2048) / block_flops(512)); the full trunk would take ~1 h on the host."""
        n = 512
        g = torch.Generator().manual_seed(0)
        z = torch.randn(1, n, n, 128, generator=g)
        s = torch.randn(1, n, 384, generator=g)
        tok = token_mask(n, n // 20, "cpu")
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}
        fn = lambda: oracle.pairformer_block(s, z, tok, params, triatt_row_chunk=64)  # noqa: E731
        frac = block_flops(n) / (len(self.blocks) * block_flops(self.n))
        return fn, frac, (f"oracle.pairformer_block fp32 at N={n}, scaled to {len(self.blocks)} blocks at "
                          f"N={self.n} by algorithmic flops")


class OpmWorkload(Workload):
    """Config 3: fused OuterProductMean, m [1,1024,512,64] bf16, seeded 20% of rows masked, added into z."""

    def __init__(self, device, n: int = 512, S: int = 1024, seed: int = 0):
        from .outer_product_mean import OuterProductMeanHip

        self.n, self.S = n, S
        self.name = f"opm_s{S}_n{n}"
        self.metric = f"ms per fused OuterProductMean at S={S}, N={n} bf16"
        torch.manual_seed(seed)
        self.module = init_module(OuterProductMeanHip(64, 32, 128), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.m_cpu = torch.randn(1, S, n, 64, generator=g).to(torch.bfloat16)
        rows = torch.rand(S, generator=torch.Generator().manual_seed(seed)) >= 0.2
        self.s_valid = int(rows.sum())
        self.mask_cpu = rows[None, :, None].expand(1, S, n).contiguous()
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.m = self.m_cpu.to(device)
        self.mask3, self.mean_rows = _ops.opm_mask3(self.mask_cpu.to(device), 1, S, n)
        self.z = self.z_cpu.to(device)
        self.ws = _ops.workspace(_ops.opm_workspace_bytes(1, S, n), device)
        self.params = self.module.prepared_params()
        self.config = {"workload": self.name, "S": S, "N": n, "c_m": 64, "c_hidden": 32, "c_out": 128,
                       "valid_rows": self.s_valid, "residual": True}
        self.flops = (2.0 * n * n * 1024 * self.s_valid + 2.0 * n * n * 1024 * 128
                      + 2.0 * self.s_valid * n * 64 * 64)

    def step(self) -> None:
        _ops.launch_opm(self.m, self.mask3, self.mean_rows, *self.params, out=self.z, z_res=self.z, ws=self.ws)

    def cpu_sample(self, oracle):
        rows = 64
        m = self.m_cpu.float()
        mask = self.mask_cpu
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}

        def fn():
            # the oracle's i-chunked loop, stopped after the first `rows` output rows
            return oracle.outer_product_mean(m, mask, params, i_chunk=rows, i_stop=rows)

        return fn, rows / self.n, f"oracle.outer_product_mean fp32 on {rows} of {self.n} output rows"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        n, S = self.n, self.S
        if kernel == "opm_fused":
            return ("mfma", 2.0 * n * n * 1024 * self.s_valid + 2.0 * n * n * 1024 * 128)
        if kernel == "opm_proj":
            return ("hbm", float(self.s_valid * n * 64 * 2 + 2 * S * n * 32 * 2))
        if kernel == "opm_rows":
            return ("hbm", float(S * n))
        if kernel == "opm_wo_tiles":  # proj_o weight [128][1024] read and written in fragment order
            return ("hbm", float(2 * 128 * 1024 * 2))
        raise KeyError(kernel)


class PwaWorkload(Workload):
    """MSA module shape: PairWeightedAveraging, m [1,1024,512,64] bf16, z [1,512,512,128], trailing
    10% of tokens padded, residual into m (m += PWA(m, z, pair mask))."""

    def __init__(self, device, n: int = 512, S: int = 1024, seed: int = 0):
        from .pair_weighted_averaging import PairWeightedAveraging

        self.n, self.S = n, S
        self.name = f"pwa_s{S}_n{n}"
        self.metric = f"ms per PairWeightedAveraging at S={S}, N={n} bf16"
        torch.manual_seed(seed)
        self.module = init_module(PairWeightedAveraging(64, 128, 32, 8), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.m_cpu = torch.randn(1, S, n, 64, generator=g).to(torch.bfloat16)
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.n_pad = n // 10
        tok = token_mask(n, self.n_pad, "cpu")
        self.mask_cpu = tok[:, :, None] & tok[:, None, :]
        self.m = self.m_cpu.to(device)
        self.z = self.z_cpu.to(device)
        self.mask = _ops.mask_u8(self.mask_cpu.to(device))
        self.ws = _ops.workspace(_ops.pwa_workspace_bytes(1, S, n, 64, 32, 8), device)
        self.params = self.module.prepared_params()
        self.config = {"workload": self.name, "S": S, "N": n, "c_m": 64, "c_z": 128, "c_h": 32, "heads": 8,
                       "padded_tokens": self.n_pad, "residual": True}
        # v, g projections + per-head averaging + output projection + bias
        self.flops = (2.0 * S * n * 64 * 512 + 2.0 * 8 * n * n * S * 32 + 2.0 * S * n * 256 * 64
                      + 2.0 * n * n * 128 * 8)

    def step(self) -> None:
        _ops.launch_pwa(self.m, self.z, self.mask, *self.params, self.m, 8, residual=True, ws=self.ws)

    def cpu_sample(self, oracle):
        rows = 16
        m = self.m_cpu[:, :rows].float()
        z = self.z_cpu.float()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}

        def fn():
            return oracle.pair_weighted_averaging(m, z, self.mask_cpu, params, num_heads=8, c_h=32)

        return fn, rows / self.S, f"oracle.pair_weighted_averaging fp32 on {rows} of {self.S} MSA rows"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        n, S = self.n, self.S
        npad = -(-n // 256) * 256
        if kernel == "pwa_fused":
            # sum_j w[h,i,j] v[s,j,h,:] over the valid keys (every head and MSA row) and the
            # output projection (g * o) Wo^T
            return ("mfma", 2.0 * 8 * n * n * S * 32 + 2.0 * S * n * 256 * 64)
        if kernel == "pwa_weights":
            # reads z, writes the 8 weight rows (bf16)
            return ("hbm", float(n * n * 128 * 2 + 8 * n * npad * 2))
        if kernel == "pwa_proj":
            # reads m, writes v^T and g (256 channels each)
            return ("hbm", float(S * n * 64 * 2 + 2 * S * npad * 256 * 2))
        if kernel == "fold_ln":  # w_z (8 rows); w_m and w_g (256 rows of width 64 each, one launch)
            return fold_kernel_work(kernel, 2, 8, 512)
        raise KeyError(kernel)


class PairMixerWorkload(Workload):
    """The reference trunk's layer (PairMixerLayer: TriMulOut, TriMulIn, Transition_z) at N=768 bf16,
    trailing 10% of tokens padded, in place."""

    cpu_warmup = 0
    cpu_calls = 1

    def __init__(self, device, n: int = 768, seed: int = 0):
        from .pairmixer import PairMixerLayerHip

        self.n = n
        self.name = f"pairmixer_layer_n{n}"
        self.metric = f"ms per PairMixer layer at N={n} bf16"
        torch.manual_seed(seed)
        self.layer = init_module(PairMixerLayerHip(384, 128), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.n_pad = n // 10
        self.tok_cpu = token_mask(n, self.n_pad, "cpu")
        self.pm_cpu = self.tok_cpu[:, :, None] & self.tok_cpu[:, None, :]
        self.z = self.z_cpu.to(device)
        self.z_tail = torch.zeros(self.z.shape, dtype=torch.int8, device=device)
        self.pm = self.pm_cpu.to(device)
        self.config = {"workload": self.name, "N": n, "c_z": 128, "batch": 1, "padded_tokens": self.n_pad,
                       "residual_stream": "bf16 + int8 tail"}
        trimul = 2.0 * n * n * 128 * 6 * 128 + 2.0 * 128 * n ** 3
        self.flops = 2 * trimul + 2.0 * n * n * 128 * 12 * 128

    def step(self) -> None:
        self.layer.forward_(None, self.z, self.pm, self.z_tail)

    def cpu_sample(self, oracle):
        params = {k: v.detach().cpu() for k, v in self.layer.state_dict().items()}
        z = self.z_cpu.float()
        s = torch.zeros(1, self.n, 384)  # passes through the layer

        def fn():
            return oracle.pairmixer_layer(s, z, self.pm_cpu, params)

        return fn, 1.0, f"oracle.pairmixer_layer fp32, full N={self.n}"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        w = trimul_kernel_work(kernel, 1, self.n)
        if w is not None:
            return w
        if kernel == "transition_pair":
            return ("mfma", 2.0 * self.n * self.n * 128 * 12 * 128)
        if kernel == "fold_ln":  # transition fc1 and fc2 (512 rows each, one launch)
            return fold_kernel_work(kernel, 1, 1024)
        raise KeyError(kernel)


class PairMixerMsaWorkload(Workload):
    """The reference MSA-module layer (PairMixerMSALayer) at S=1024, N=512 bf16: PWA, MSA transition,
    OPM (20% of MSA rows masked), TriMulOut, TriMulIn, Transition_z, in place."""

    cpu_warmup = 0
    cpu_calls = 1

    def __init__(self, device, n: int = 512, S: int = 1024, seed: int = 0):
        from .pairmixer import PairMixerMSALayerHip

        self.n, self.S = n, S
        self.name = f"pairmixer_msa_layer_s{S}_n{n}"
        self.metric = f"ms per PairMixer MSA layer at S={S}, N={n} bf16"
        torch.manual_seed(seed)
        self.layer = init_module(PairMixerMSALayerHip(384, 64, 128, 0.15, 0.25), seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.m_cpu = torch.randn(1, S, n, 64, generator=g).to(torch.bfloat16)
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.n_pad = n // 10
        tok = token_mask(n, self.n_pad, "cpu")
        self.pm_cpu = tok[:, :, None] & tok[:, None, :]
        rows = torch.rand(S, generator=torch.Generator().manual_seed(seed)) >= 0.2
        self.msa_mask_cpu = rows[None, :, None] & tok[:, None, :]
        self.m = self.m_cpu.to(device)
        self.z = self.z_cpu.to(device)
        self.pm = self.pm_cpu.to(device)
        self.msa_mask = self.msa_mask_cpu.to(device)
        self.s_valid = int(rows.sum())
        self.z_tail = torch.zeros(self.z.shape, dtype=torch.int8, device=device)
        self.m_tail = torch.zeros(self.m.shape, dtype=torch.int8, device=device)
        self.config = {"workload": self.name, "S": S, "N": n, "c_m": 64, "c_z": 128, "batch": 1,
                       "padded_tokens": self.n_pad, "valid_msa_rows": self.s_valid,
                       "residual_stream": "bf16 + int8 tail"}
        pwa = 2.0 * S * n * 64 * 512 + 2.0 * 8 * n * n * S * 32 + 2.0 * S * n * 256 * 64
        msa_tr = 2.0 * S * n * 64 * 12 * 64
        opm = 2.0 * n * n * 1024 * self.s_valid + 2.0 * n * n * 1024 * 128
        trimul = 2.0 * n * n * 128 * 6 * 128 + 2.0 * 128 * n ** 3
        self.flops = pwa + msa_tr + opm + 2 * trimul + 2.0 * n * n * 128 * 12 * 128

    def step(self) -> None:
        self.layer.forward_(None, self.z, self.m, self.pm, self.msa_mask, z_tail=self.z_tail, m_tail=self.m_tail)

    def cpu_sample(self, oracle):
        """Every op of the layer, each on a bounded slice scaled to the full layer: PWA and the MSA
        transition on 16 of S MSA rows (both are independent per MSA row), the OPM on 64 of N output
        rows, the two triangle multiplications and the pair transition at full size.  The callable
        returns that extrapolated time in seconds (fraction None)."""
        rows, opm_rows = 16, 64
        params = {k: v.detach().cpu() for k, v in self.layer.state_dict().items()}

        def sub(prefix):
            return {k[len(prefix) + 1:]: v for k, v in params.items() if k.startswith(prefix + ".")}

        m = self.m_cpu.float()
        z = self.z_cpu.float()
        msa_mask = self.msa_mask_cpu

        def fn():
            t0 = time.perf_counter()
            mm = m[:, :rows] + oracle.pair_weighted_averaging(m[:, :rows], z, self.pm_cpu,
                                                               sub("pair_weighted_averaging"))
            mm = mm + oracle.transition(mm, sub("msa_transition"))
            t1 = time.perf_counter()
            oracle.outer_product_mean(m, msa_mask, sub("outer_product_mean"), i_chunk=opm_rows, i_stop=opm_rows)
            t2 = time.perf_counter()
            zz = z + oracle.trimul(z, self.pm_cpu, sub("tri_mul_out"), "outgoing")
            zz = zz + oracle.trimul(zz, self.pm_cpu, sub("tri_mul_in"), "incoming")
            zz = zz + oracle.transition(zz, sub("z_transition"))
            t3 = time.perf_counter()
            return (t1 - t0) * self.S / rows + (t2 - t1) * self.n / opm_rows + (t3 - t2)

        return fn, None, (f"fp32 oracle ops: PWA + MSA transition on {rows} of {self.S} MSA rows, "
                          f"OPM on {opm_rows} of {self.n} output rows, TriMulOut + TriMulIn + Transition_z "
                          f"at full N; each part scaled to the full layer")

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        n, S = self.n, self.S
        w = trimul_kernel_work(kernel, 1, n)
        if w is not None:
            return w
        if kernel == "transition_pair":
            return ("mfma", 2.0 * n * n * 128 * 12 * 128)
        if kernel == "opm_fused":
            return ("mfma", 2.0 * n * n * 1024 * self.s_valid + 2.0 * n * n * 1024 * 128)
        if kernel == "opm_proj":
            return ("hbm", float(self.s_valid * n * 64 * 2 + 2 * S * n * 32 * 2))
        if kernel == "opm_rows":
            return ("hbm", float(S * n))
        if kernel == "opm_wo_tiles":
            return ("hbm", float(2 * 128 * 1024 * 2))
        if kernel in ("pwa_weights", "pwa_proj", "pwa_fused"):
            return PwaWorkload.kernel_work(self, kernel)
        if kernel == "transition_msa":
            return ("mfma", 2.0 * S * n * 64 * 12 * 64)
        if kernel == "fold_ln":  # PWA (2 launches), MSA transition and pair transition (one launch each)
            return fold_kernel_work(kernel, 4, 8 + 1024, 512 + 512)
        raise KeyError(kernel)


class PairMixerTrunkWorkload(Workload):
    """The reference's sequence trunk from its initial embeddings on (PairMixerSequenceEmbedder.forward,
    pairmixer.py:275-296) at N=768 (76 padded tokens), S=1024 MSA rows (20 % masked): one pass
    (num_steps_recycle = 0) = the recycling updates, the MSA module (input embedding + 4 MSA layers) and the
    48-layer PairMixer stack, z carried as one bf16 + int8-tail stream."""

    cpu_warmup = 0
    cpu_calls = 1

    def __init__(self, device, n: int = 768, S: int = 1024, blocks: int = 48, msa_blocks: int = 4,
                 seed: int = 0):
        from .pairmixer import NUM_TOKENS, PairMixerTrunkHip

        self.n, self.S, self.blocks, self.msa_blocks = n, S, blocks, msa_blocks
        self.name = f"pairmixer_trunk{blocks}_msa{msa_blocks}_s{S}_n{n}"
        self.metric = f"ms per PairMixer trunk pass ({msa_blocks} MSA + {blocks} layers) at S={S}, N={n} bf16"
        torch.manual_seed(seed)
        self.module = init_module(PairMixerTrunkHip(384, 128, 455, msa_blocks=msa_blocks, num_blocks=blocks),
                                  seed).to(device).eval()
        g = torch.Generator().manual_seed(seed)
        self.n_pad = n // 10
        tok = token_mask(n, self.n_pad, "cpu")
        rows = torch.rand(S, generator=g) >= 0.2
        self.s_valid = int(rows.sum())
        self.s_init = torch.randn(1, n, 384, generator=g).to(torch.bfloat16).to(device)
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.z_init = self.z_cpu.to(device)
        self.emb = torch.randn(1, n, 455, generator=g).to(device)
        aa = torch.randint(0, NUM_TOKENS, (1, S, n), generator=g)
        self.feats_cpu = {
            "msa": torch.nn.functional.one_hot(aa, NUM_TOKENS).float(),
            "has_deletion": (torch.rand(1, S, n, generator=g) < 0.1).float(),
            "deletion_value": torch.rand(1, S, n, generator=g),
            "msa_paired": (torch.rand(1, S, n, generator=g) < 0.5).float(),
            "msa_mask": rows[None, :, None] & tok[:, None, :],
            "token_pad_mask": tok,
        }
        self.feats = {k: v.to(device) for k, v in self.feats_cpu.items()}
        self.pm_cpu = tok[:, :, None] & tok[:, None, :]
        self.config = {"workload": self.name, "N": n, "S": S, "msa_blocks": msa_blocks, "blocks": blocks,
                       "num_steps_recycle": 0, "c_z": 128, "c_m": 64, "c_s": 384, "batch": 1,
                       "padded_tokens": self.n_pad, "valid_msa_rows": self.s_valid,
                       "residual_stream": "bf16 + int8 tail"}
        P = n * n
        trimul = 2.0 * P * 128 * 6 * 128 + 2.0 * 128 * n ** 3
        layer = 2 * trimul + 2.0 * P * 128 * 12 * 128
        pwa = 2.0 * S * n * 64 * 512 + 2.0 * 8 * n * n * S * 32 + 2.0 * S * n * 256 * 64
        msa_tr = 2.0 * S * n * 64 * 12 * 64
        opm = 2.0 * P * 1024 * self.s_valid + 2.0 * P * 1024 * 128
        recycle = 2.0 * P * 128 * 128 + 2.0 * n * 384 * 384
        self.flops = blocks * layer + msa_blocks * (pwa + msa_tr + opm + layer) + recycle

    def step(self) -> None:
        self.module(self.s_init, self.z_init, self.emb, self.feats, 0)

    def cpu_sample(self, oracle):
        """fp32 oracle ops, each timed once and scaled to the pass: one PairMixer layer at full N (x 48, and
        the same three z updates inside each of the 4 MSA layers), PWA + MSA transition on 16 of S MSA rows
        and the OPM on 64 of N output rows (x 4, scaled to the full sizes), the two recycling updates."""
        rows, opm_rows = 16, 64
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}

        def sub(prefix):
            return {k[len(prefix) + 1:]: v for k, v in params.items() if k.startswith(prefix + ".")}

        z = self.z_cpu.float()
        s = self.s_init.float().cpu()
        msa = sub("msa_module")
        layer0 = sub("msa_module.layers.0")

        def fn():
            t0 = time.perf_counter()
            oracle.ln_linear(z, z, params, "z_norm", "z_recycle")
            oracle.ln_linear(s, s, params, "s_norm", "s_recycle")
            f = self.feats_cpu
            m = oracle.msa_embed(f["msa"][:, :rows], f["has_deletion"][:, :rows], f["deletion_value"][:, :rows],
                                 f["msa_paired"][:, :rows], self.emb.cpu(), msa)
            t1 = time.perf_counter()
            m = m + oracle.pair_weighted_averaging(m, z, self.pm_cpu, {k[len("pair_weighted_averaging") + 1:]: v
                                                                       for k, v in layer0.items()
                                                                       if k.startswith("pair_weighted_averaging.")})
            m = m + oracle.transition(m, {k[len("msa_transition") + 1:]: v for k, v in layer0.items()
                                          if k.startswith("msa_transition.")})
            t2 = time.perf_counter()
            m_full = torch.randn(1, self.S, self.n, 64)
            oracle.outer_product_mean(m_full, f["msa_mask"], {k[len("outer_product_mean") + 1:]: v
                                                              for k, v in layer0.items()
                                                              if k.startswith("outer_product_mean.")},
                                      i_chunk=opm_rows, i_stop=opm_rows)
            t3 = time.perf_counter()
            oracle.pairmixer_layer(s, z, self.pm_cpu, sub("pairmixer_module.layers.0"))
            t4 = time.perf_counter()
            return ((t1 - t0) + self.msa_blocks * ((t2 - t1) * self.S / rows + (t3 - t2) * self.n / opm_rows)
                    + (self.blocks + self.msa_blocks) * (t4 - t3))

        return fn, None, (f"fp32 oracle ops scaled to one pass: PairMixer layer at full N x "
                          f"{self.blocks + self.msa_blocks}; PWA + MSA transition on {rows} of {self.S} rows and "
                          f"OPM on {opm_rows} of {self.n} output rows x {self.msa_blocks}; recycling updates")

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        n, S, L = self.n, self.S, self.blocks + self.msa_blocks
        w = trimul_kernel_work(kernel, 1, n)
        if w is not None:
            return w
        if kernel == "transition_pair":
            return ("mfma", 2.0 * n * n * 128 * 12 * 128)
        if kernel == "opm_fused":
            return ("mfma", 2.0 * n * n * 1024 * self.s_valid + 2.0 * n * n * 1024 * 128)
        if kernel == "opm_wo_tiles":
            return ("hbm", float(2 * 128 * 1024 * 2))
        if kernel in ("pwa_weights", "pwa_proj", "pwa_fused"):
            return PwaWorkload.kernel_work(self, kernel)
        if kernel == "transition_msa":
            return ("mfma", 2.0 * S * n * 64 * 12 * 64)
        if kernel == "pair_ln_linear":
            return ("hbm", float(n * n * 128 * (2 + 3 + 3)))   # x, base + tail in; out + tail
        if kernel == "msa_embed":
            return ("hbm", float(S * n * (33 + 3) * 4 + S * n * 64 * 3))
        if kernel == "fold_ln":   # launches: pair transitions (L), PWA (2) + MSA transition per MSA layer, z recycle
            mb = self.msa_blocks
            return fold_kernel_work(kernel, L + 3 * mb + 1, L * 1024 + 8 * mb + 128, mb * 1024)
        raise KeyError(kernel)


class SwaWorkload(Workload):
    """The denoiser's atom transformer attention (AttentionPairBiasSlidingWindow as AttentionLayer builds it,
    transformer.py:96-105: initial_norm=False): NA = 6144 atoms (NW = 192 windows of W = 32, H = 128 keys),
    c_s = 128, 4 heads, c_z = 16, multiplicity M = 8, trailing 40 atoms padded."""

    def __init__(self, device, nw: int = 192, mult: int = 8, seed: int = 0, fp32: bool = False):
        from .attention_pair_bias import AttentionPairBiasSlidingWindow

        self.nw, self.mult, self.fp32 = nw, mult, fp32
        self.na = nw * 32
        self.dtype = "f32" if fp32 else "bf16"
        self.name = f"swa_na{self.na}_m{mult}" + ("_f32" if fp32 else "")
        self.metric = f"ms per sliding-window pair-bias attention at {self.na} atoms, M={mult} {self.dtype}"
        torch.manual_seed(seed)
        self.module = init_module(AttentionPairBiasSlidingWindow(128, 16, 4, initial_norm=False), seed)
        self.module = self.module.to(device).eval()
        g = torch.Generator().manual_seed(seed)
        dt = torch.float32 if fp32 else torch.bfloat16
        self.s_cpu = torch.randn(mult * nw, 32, 128, generator=g).to(dt)
        self.z_cpu = torch.randn(1, nw, 32, 128, 16, generator=g).to(dt)
        mask = torch.ones(1, self.na, dtype=torch.bool)
        mask[:, -40:] = False
        self.mask_cpu = mask.view(nw, 32)
        self.s = self.s_cpu.to(device)
        self.z = self.z_cpu.to(device)
        self.mask = _ops.mask_u8(self.mask_cpu.to(device))
        self.out = torch.empty_like(self.s)
        ws_bytes = (_ops.swa_f32_workspace_bytes if fp32 else _ops.swa_workspace_bytes)(1, mult, nw, 32, 128, 128, 4)
        self.ws = _ops.workspace(ws_bytes, device)
        self.params = self.module.prepared_params_f32() if fp32 else self.module.prepared_params()
        self.launch = _ops.launch_swa_f32 if fp32 else _ops.launch_swa
        self.config = {"workload": self.name, "atoms": self.na, "windows": nw, "window_queries": 32,
                       "window_keys": 128, "c_s": 128, "c_z": 16, "heads": 4, "multiplicity": mult,
                       "initial_norm": False, "padded_atoms": 40}
        rows = mult * self.na
        self.flops = 2.0 * rows * 128 * 128 * 5 + 2.0 * mult * nw * 4 * 32 * 128 * 32 * 2 + 2.0 * nw * 32 * 128 * 16 * 4

    def step(self) -> None:
        self.launch(self.s, self.z, self.mask, *self.params, self.out, 4, multiplicity=self.mult, ws=self.ws)

    def cpu_sample(self, oracle):
        s = self.s_cpu[: self.nw].float()   # copy 0 of M (copies are independent)
        z = self.z_cpu.float()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}

        def fn():
            return oracle.attention_pair_bias_sliding_window(s, z, self.mask_cpu, params, 4, initial_norm=False)

        return fn, 1.0 / self.mult, f"oracle.attention_pair_bias_sliding_window fp32 on 1 of {self.mult} copies"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        rows = self.mult * self.na
        if self.fp32:
            if kernel == "f32_proj_qkvg":
                return ("mfma_f32", 4 * 2.0 * rows * 128 * 128)
            if kernel == "f32_proj_o":
                return ("mfma_f32", 2.0 * rows * 128 * 128)
            if kernel == "f32_swa_pair_bias":   # reads z, writes the 4-head bias
                return ("hbm", float(self.nw * 32 * 128 * (16 + 4) * 4))
            if kernel == "f32_swa_attention":   # QK^T and PV over the 128-key window, every copy and head
                return ("mfma_f32", 2.0 * 2 * rows * 128 * 128)
            raise KeyError(kernel)
        tok = rows * 128 * 2
        bias = self.nw * 4 * 32 * 128 * 2
        if kernel == "swa_attn":
            # reads q, k, v, g and the bias once, writes g*o
            return ("hbm", float(5 * tok + bias))
        if kernel == "swa_pair_bias":
            return ("hbm", float(self.nw * 32 * 128 * 16 * 2 + bias))
        if kernel == "swa_proj_qkvg":   # the four per-atom projections in one launch: read s, write q, k, v^T, g
            return ("hbm", float(5 * tok + 4 * 128 * 128 * 2))
        if kernel == "swa_proj_o":
            return ("hbm", float(2 * tok + 128 * 128 * 2))
        raise KeyError(kernel)


class ApbWorkload(Workload):
    """Config 2: pair-bias attention, s [8,512,384] bf16, z [8,512,512,128], 16 heads of 24, last 51 keys
    masked (initial_norm=True); with ``mult`` > 1 the denoiser form: B=1, M copies sharing one z."""

    def __init__(self, device, n: int = 512, B: int = 8, mult: int = 1, initial_norm: bool = True, seed: int = 0,
                 fp32: bool = False):
        from .attention_pair_bias import AttentionPairBias

        self.n, self.B, self.mult, self.fp32 = n, B, mult, fp32
        self.dtype = "f32" if fp32 else "bf16"
        self.name = f"apb_b{B}_m{mult}_n{n}" + ("" if initial_norm else "_nonorm") + ("_f32" if fp32 else "")
        self.metric = f"ms per pair-bias attention at B={B}, M={mult}, N={n} {self.dtype}"
        torch.manual_seed(seed)
        self.module = init_module(AttentionPairBias(384, 128, 16, initial_norm=initial_norm), seed).to(device)
        self.module = self.module.eval()
        g = torch.Generator().manual_seed(seed)
        dt = torch.float32 if fp32 else torch.bfloat16
        self.s_cpu = torch.randn(B * mult, n, 384, generator=g).to(dt)
        self.z_cpu = torch.randn(B, n, n, 128, generator=g).to(dt)
        self.mask_cpu = torch.ones(B, n, dtype=torch.bool)
        self.mask_cpu[:, n - n // 10:] = False
        self.initial_norm = initial_norm
        self.s = self.s_cpu.to(device)
        self.z = self.z_cpu.to(device)
        self.mask = _ops.mask_u8(self.mask_cpu.to(device))
        self.out = torch.empty_like(self.s)
        ws_bytes = (_ops.apb_f32_workspace_bytes if fp32 else _ops.apb_workspace_bytes)(B, mult, n, 384, 16)
        self.ws = _ops.workspace(ws_bytes, device)
        self.params = self.module.prepared_params_f32() if fp32 else self.module.prepared_params()
        self.launch = _ops.launch_apb_f32 if fp32 else _ops.launch_apb
        self.config = {"workload": self.name, "batch": B, "multiplicity": mult, "N": n, "c_s": 384, "c_z": 128,
                       "heads": 16, "head_dim": 24, "masked_keys": n // 10, "initial_norm": initial_norm}
        rows = B * mult * n
        self.flops = (2.0 * rows * 384 * 384 * 5 + 2.0 * B * n * n * 128 * 16
                      + 2.0 * 2 * B * mult * n * n * 384)

    def step(self) -> None:
        self.launch(self.s, self.z, self.mask, *self.params, self.out, 16, self.mult, ws=self.ws)

    def cpu_sample(self, oracle):
        s = self.s_cpu[: self.mult].float()   # batch element 0 with its M copies
        z = self.z_cpu[:1].float()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}

        def fn():
            return oracle.attention_pair_bias(s, z, self.mask_cpu[:1], params, 16, multiplicity=self.mult,
                                              initial_norm=self.initial_norm)

        return fn, 1.0 / self.B, f"oracle.attention_pair_bias fp32 on batch element 1 of {self.B}"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        n, B, M = self.n, self.B, self.mult
        if self.fp32:
            rows = B * M * n
            if kernel == "f32_proj_qkvg":
                return ("mfma_f32", 4 * 2.0 * rows * 384 * 384)
            if kernel == "f32_proj_o":
                return ("mfma_f32", 2.0 * rows * 384 * 384)
            if kernel == "f32_layernorm":
                return ("hbm", float(2 * rows * 384 * 4))
            if kernel == "f32_pair_bias":   # reads z, writes the 16-head bias
                return ("hbm", float(B * n * n * (128 + 16) * 4))
            if kernel == "f32_attention":   # QK^T and PV: 4 N^2 c_s per copy
                return ("mfma_f32", 4.0 * B * M * n * n * 384)
            raise KeyError(kernel)
        np_ = -(-n // 32) * 32
        tok = B * M * np_ * 384 * 2
        if kernel == "apb_pair_bias":
            return ("hbm", float(B * n * n * 128 * 2 + B * 16 * np_ * np_ * 2))
        if kernel == "apb_flash":
            # reads q, k, v, g and the bias, writes g*o; the QK^T / PV products are 4 N^2 c_s flops per copy
            return ("hbm", float(5 * tok + B * 16 * np_ * np_ * 2))
        if kernel == "apb_proj_qkvg":   # the four token projections in one launch
            return ("mfma", 4 * 2.0 * B * M * np_ * 384 * 384)
        if kernel in ("apb_proj_o", "token_layernorm"):
            return ("hbm", float(2 * tok + 384 * 384 * 2))
        if kernel == "fold_ln":
            return fold_kernel_work(kernel, 1, 16)
        raise KeyError(kernel)


class DistogramWorkload(Workload):
    """The trunk's distogram head (DistogramModule, token_z 128, 64 bins) on z [1,768,768,128] bf16."""

    def __init__(self, device, n: int = 768, bins: int = 64, seed: int = 0):
        from .glue import DistogramModule

        self.n, self.bins = n, bins
        self.name = f"distogram_n{n}_bins{bins}"
        self.metric = f"ms per distogram head at N={n}, {bins} bins bf16"
        torch.manual_seed(seed)
        self.module = init_module(DistogramModule(128, bins), seed).to(device)
        g = torch.Generator().manual_seed(seed)
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(torch.bfloat16)
        self.z = self.z_cpu.to(device)
        self.out = torch.empty(1, n, n, bins, dtype=torch.bfloat16, device=device)
        self.params = self.module.prepared_params()
        self.config = {"workload": self.name, "N": n, "c_z": 128, "num_bins": bins}
        self.flops = 2.0 * n * n * 128 * bins

    def step(self) -> None:
        _ops.launch_distogram(self.z, *self.params, self.out)

    def cpu_sample(self, oracle):
        z = self.z_cpu.float()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}
        return (lambda: oracle.distogram(z, params)), 1.0, f"oracle.distogram fp32, full N={self.n}"

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        if kernel == "distogram":
            # reads z once (each unordered pair's two rows), writes both orders of the output
            return ("hbm", float(self.n * self.n * (128 + self.bins) * 2))
        raise KeyError(kernel)


class PairCondWorkload(Workload):
    """The denoiser's PairwiseConditioning (token_z = rel = a_z = 128, 2 transitions of hidden 256) at N=768."""

    def __init__(self, device, n: int = 768, seed: int = 0, fp32: bool = False):
        from .glue import PairwiseConditioning

        self.n, self.fp32 = n, fp32
        self.dtype = "f32" if fp32 else "bf16"
        self.name = f"pair_cond_n{n}" + ("_f32" if fp32 else "")
        self.metric = f"ms per pairwise conditioning at N={n} {self.dtype}"
        torch.manual_seed(seed)
        self.module = init_module(PairwiseConditioning(128, 128), seed).to(device)
        g = torch.Generator().manual_seed(seed)
        dt = torch.float32 if fp32 else torch.bfloat16
        self.z_cpu = torch.randn(1, n, n, 128, generator=g).to(dt)
        self.rel_cpu = torch.randn(1, n, n, 128, generator=g).to(dt)
        self.z = self.z_cpu.to(device)
        self.rel = self.rel_cpu.to(device)
        self.config = {"workload": self.name, "N": n, "token_z": 128, "rel_pos": 128, "a_z": 128,
                       "transitions": 2, "transition_hidden": 256}
        self.flops = 2.0 * n * n * 256 * 128 + 2 * 2.0 * n * n * 128 * 768

    def step(self) -> None:
        self.module(self.z, self.rel)

    def cpu_sample(self, oracle):
        rows = 64
        z = self.z_cpu[:, :rows].float()
        rel = self.rel_cpu[:, :rows].float()
        params = {k: v.detach().cpu() for k, v in self.module.state_dict().items()}
        return ((lambda: oracle.pairwise_conditioning(z, rel, params)), rows / self.n,
                f"oracle.pairwise_conditioning fp32 on {rows} of {self.n} rows")

    def kernel_work(self, kernel: str) -> tuple[str, float]:
        P = self.n * self.n
        if self.fp32:
            if kernel == "f32_pair_cond_layernorm":   # reads both inputs, writes the normalised concatenation
                return ("hbm", float(P * 256 * 4 * 2))
            if kernel == "f32_layernorm":
                return ("hbm", float(P * 128 * 4 * 2))
            if kernel == "f32_pair_cond_proj":
                return ("mfma_f32", 2.0 * P * 256 * 128)
            if kernel == "f32_transition_swiglu":   # fc1 and fc2, 128 -> 256 each
                return ("mfma_f32", 2.0 * 2 * P * 128 * 256)
            if kernel == "f32_transition_out":
                return ("mfma_f32", 2.0 * P * 256 * 128)
            raise KeyError(kernel)
        if kernel == "pair_cond_proj":
            return ("hbm", float(P * (256 + 128) * 2))
        if kernel == "transition_pair":
            return ("mfma", 2.0 * P * 128 * 768)
        if kernel == "fold_ln":  # the projection (128 rows of width 256) and fc1, fc2 of both transitions
            return fold_kernel_work(kernel, 5, 4 * 256, rows256=128)
        raise KeyError(kernel)


def make(op: str, device, n: int | None = None) -> Workload:
    if op == "opm":
        return OpmWorkload(device, n or 512)
    if op == "pwa":
        return PwaWorkload(device, n or 512)
    if op == "swa":
        return SwaWorkload(device)
    if op == "apb":
        return ApbWorkload(device, n or 512)
    if op == "apb_nonorm":   # config 2 in the denoiser's setting (initial_norm=False)
        return ApbWorkload(device, n or 512, initial_norm=False)
    if op == "apb_denoiser":
        return ApbWorkload(device, n or 768, B=1, mult=8, initial_norm=False)
    # the denoiser's ops on the fp32 path (the reference runs its denoiser with autocast off)
    if op == "apb_denoiser_f32":
        return ApbWorkload(device, n or 768, B=1, mult=8, initial_norm=False, fp32=True)
    if op == "swa_f32":
        return SwaWorkload(device, fp32=True)
    if op == "pair_cond_f32":
        return PairCondWorkload(device, n or 768, fp32=True)
    if op == "distogram":
        return DistogramWorkload(device, n or 768)
    if op == "pair_cond":
        return PairCondWorkload(device, n or 768)
    if op == "pairmixer":
        return PairMixerWorkload(device, n or 768)
    if op == "pairmixer_msa":
        return PairMixerMsaWorkload(device, n or 512)
    if op == "block":
        return BlockWorkload(device, n or 768)
    if op == "block_bf16stream":   # the same block with plain bf16 residual streams (no tails)
        return BlockWorkload(device, n or 768, tails=False)
    if op == "config1":            # the reference's CPU case: N = 64, fp32 in/out
        return Config1Workload(device, n or 64)
    if op == "pairmixer_trunk":    # recycling + MSA module (4 layers) + 48 PairMixer layers, one pass
        return PairMixerTrunkWorkload(device, n or 768)
    if op == "trunk":              # config 5: 48 blocks at N = 2048
        return TrunkWorkload(device, n or 2048)
    if op in ("triatt_start", "triatt_end"):
        return TriAttWorkload(device, op == "triatt_start", n or 768)
    if op in ("trimul_out", "trimul_in"):
        return TriMulWorkload(device, "outgoing" if op == "trimul_out" else "incoming", n or 768)
    raise ValueError(f"unknown bench op {op!r}")


__all__ = ["make", "measured_traffic", "Workload", "token_mask", "init_module", "math"]
