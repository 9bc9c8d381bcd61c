"""The PairMixer trunk above the layers on the GPU vs the fp32 CPU oracle.

Covers the recycling updates (``bioemu_pair_ln_linear_fwd`` / ``bioemu_token_ln_linear_fwd``), the MSA input
embedding (``bioemu_msa_embed_fwd``), ``PairMixerModuleHip`` (the layer stack), ``PairMixerMSAModuleHip``
and the recycling loop of ``PairMixerTrunkHip`` (pairmixer.py:275-296, :352-370, :553-611).  Streams carry
int8 tails, so the bf16 bound (max-abs 2e-2, rel-L2 1e-2) holds on every valid element; the MSA embedding is
fp32 arithmetic and is held to ~2^-15 relative (its output is the bf16 + tail stream).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from bioemu2_amd import _ops
from bioemu2_amd.pairmixer import NUM_TOKENS, PairMixerModuleHip, PairMixerMSAModuleHip, PairMixerTrunkHip
from bioemu2_amd.residual import join_stream, split_stream
from bioemu2_amd.workloads import init_module
from tests._helpers import max_abs, rel_l2, state

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("bf16_autocast")]


def _check(name, got, want, sel=None):
    g, w = got.float().cpu(), want.float()
    if sel is not None:
        g, w = g[sel], w[sel]
    err, rl2 = max_abs(g, w), rel_l2(g, w)
    print(f"{name}: max_abs={err:.3e} rel_l2={rl2:.3e} |want|max={w.abs().max():.2f}", flush=True)
    assert err <= 2e-2 and rl2 <= 1e-2, (name, err, rl2)


def _randn(shape, g, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).float()


def _tok(B, n, n_pad):
    tok = torch.ones(B, n, dtype=torch.bool)
    if n_pad:
        tok[:, n - n_pad:] = False
    return tok


def _feats(B, R, T, n_pad, g, device):
    tok = torch.randint(0, NUM_TOKENS, (B, R, T), generator=g)
    f = {
        "msa": torch.nn.functional.one_hot(tok, NUM_TOKENS).float(),
        "has_deletion": (torch.rand(B, R, T, generator=g) < 0.3).float(),
        "deletion_value": torch.rand(B, R, T, generator=g),
        "msa_paired": (torch.rand(B, R, T, generator=g) < 0.5).float(),
        "msa_mask": torch.rand(B, R, T, generator=g) > 0.2,
        "token_pad_mask": _tok(B, T, n_pad),
    }
    return f, {k: v.to(device) for k, v in f.items()}


@pytest.mark.parametrize("tails", [False, True])
def test_pair_ln_linear_matches_oracle(gpu_device, tails):
    g = torch.Generator().manual_seed(0)
    P = 37 * 41                                     # not a multiple of the 32-row tile
    x, base = _randn((1, 37, 41, 128), g), _randn((1, 37, 41, 128), g, 3.0)
    prm = {"z_norm.weight": 1 + 0.1 * torch.randn(128, generator=g), "z_norm.bias": 0.1 * torch.randn(128, generator=g),
           "z_recycle.weight": torch.randn(128, 128, generator=g) / 11.3}
    want = oracle.ln_linear(x, base, prm, "z_norm", "z_recycle")
    d = gpu_device
    xs = x.to(torch.bfloat16).to(d)
    w = prm["z_recycle.weight"].to(torch.bfloat16).to(d)
    nw, nb = prm["z_norm.weight"].to(d), prm["z_norm.bias"].to(d)
    if tails:
        b_hi, b_tail = split_stream(base.to(d))
        out, out_tail = torch.empty_like(b_hi), torch.empty_like(b_tail)
        _ops.launch_ln_linear(xs, nw, nb, w, b_hi, out, base_tail=b_tail, out_tail=out_tail)
        got = join_stream(out, out_tail)
        # in place on x (z = z_init + z_recycle(z_norm(z)) overwrites z)
        xi = xs.clone()
        xi_tail = torch.empty(xi.shape, dtype=torch.int8, device=d)
        _ops.launch_ln_linear(xi, nw, nb, w, b_hi, xi, base_tail=b_tail, out_tail=xi_tail)
        assert torch.equal(xi, out) and torch.equal(xi_tail, out_tail)
    else:
        out = torch.empty_like(xs)
        _ops.launch_ln_linear(xs, nw, nb, w, base.to(torch.bfloat16).to(d), out)
        # a plain bf16 output carries its own rounding (half an ulp, 2^-9 |x|, up to 3e-2 at |x| ~ 15):
        # the bound is 2e-2 on top of one bf16 ulp of the value, elementwise
        g32 = out.float().cpu()
        excess = ((g32 - want).abs() - 2.0 ** -8 * want.abs()).max().item()
        print(f"pair_ln_linear bf16 out: max excess over 1 ulp = {excess:.3e}, rel_l2={rel_l2(g32, want):.3e}",
              flush=True)
        assert excess <= 2e-2 and rel_l2(g32, want) <= 1e-2
        return
    assert P == got[0].numel() // 128
    _check(f"pair_ln_linear tails={tails}", got, want)


def test_token_ln_linear_matches_oracle(gpu_device):
    g = torch.Generator().manual_seed(1)
    x, base = _randn((2, 50, 384), g), _randn((2, 50, 384), g, 2.0)
    prm = {"s_norm.weight": 1 + 0.1 * torch.randn(384, generator=g), "s_norm.bias": 0.1 * torch.randn(384, generator=g),
           "s_recycle.weight": torch.randn(384, 384, generator=g) / 19.6}
    want = oracle.ln_linear(x, base, prm, "s_norm", "s_recycle")
    d = gpu_device
    xs = x.to(torch.bfloat16).to(d)
    b_hi, b_tail = split_stream(base.to(d))
    out, out_tail = torch.empty_like(b_hi), torch.empty_like(b_tail)
    _ops.launch_ln_linear(xs, prm["s_norm.weight"].to(d), prm["s_norm.bias"].to(d),
                          prm["s_recycle.weight"].to(torch.bfloat16).to(d), b_hi, out, base_tail=b_tail,
                          out_tail=out_tail)
    _check("token_ln_linear", join_stream(out, out_tail), want)
    assert torch.equal(b_hi, split_stream(base.to(d))[0])       # base untouched


@pytest.mark.parametrize("paired", [True, False])
def test_msa_embed_matches_oracle(gpu_device, paired):
    g = torch.Generator().manual_seed(2)
    B, R, T, E = 2, 7, 45, 455
    f, fd = _feats(B, R, T, 0, g, gpu_device)
    emb = torch.randn(B, T, E, generator=g)
    wm = torch.randn(64, NUM_TOKENS + 2 + int(paired), generator=g)
    ws = torch.randn(64, E, generator=g) / 21.0
    want = oracle.msa_embed(f["msa"], f["has_deletion"], f["deletion_value"], f["msa_paired"] if paired else None,
                            emb, {"msa_proj.weight": wm, "s_proj.weight": ws})
    m = torch.empty(B, R, T, 64, dtype=torch.bfloat16, device=gpu_device)
    m_tail = torch.empty(B, R, T, 64, dtype=torch.int8, device=gpu_device)
    _ops.launch_msa_embed(fd["msa"], fd["has_deletion"], fd["deletion_value"], fd["msa_paired"] if paired else None,
                          emb.to(gpu_device), wm.to(gpu_device), ws.to(gpu_device), m, m_tail)
    got = join_stream(m, m_tail).cpu()
    err = (got - want).abs().max().item()
    print(f"msa_embed paired={paired}: max_abs={err:.3e} |want|max={want.abs().max():.2f}", flush=True)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-5)


def _e2e(name, got, want, sel, layers):
    """A stack end to end against the oracle stack: rel-L2 at the plain bound (1e-2); max-abs at 2e-2 sqrt(layers).

    Each layer is held to the plain bound alone, on its own input, by the layer-by-layer checks.  Its error is
    the rounding of its MFMA operands (LayerNorm outputs and weights to bf16; the residual streams carry ~16
    bits and add nothing), independent from layer to layer, so end to end the errors add in quadrature:
    measured 1.3-1.6e-2 for one layer, 1.9-2.2e-2 over two and 2.4e-2 over four.  The bound 2e-2 sqrt(layers)
    is the per-layer bound grown that way; rel-L2 stays at 1e-2 (measured <= 3.9e-3 over four layers)."""
    g, w = got.float().cpu()[sel], want.float()[sel]
    err, rl2 = max_abs(g, w), rel_l2(g, w)
    bound = 2e-2 * layers ** 0.5
    print(f"{name} (end to end, {layers} layers): max_abs={err:.3e} (bound {bound:.2e}) rel_l2={rl2:.3e}",
          flush=True)
    assert rl2 <= 1e-2 and err <= bound, (name, err, rl2)


def test_pairmixer_module_is_its_layers_each_within_bound(gpu_device):
    """The module equals its layers run in order, bit for bit; every layer, fed the GPU's own input, is within
    the bf16 bound of the oracle layer; end to end against the oracle stack."""
    n, n_pad, blocks = 64, 6, 2
    d = gpu_device
    torch.manual_seed(0)
    mod = init_module(PairMixerModuleHip(384, 128, blocks), 0).to(d).eval()
    g = torch.Generator().manual_seed(3)
    s, z = _randn((1, n, 384), g), _randn((1, n, n, 128), g)
    tok = _tok(1, n, n_pad)
    pm = oracle.pair_mask_from_token_mask(tok)
    s_got, z_got = mod(s.to(d), z.to(d), pm.to(d))
    assert torch.equal(s_got.cpu(), s)
    z_cur = z.to(d)
    for i, layer in enumerate(mod.layers):
        _, z_next = layer(s.to(d), z_cur, pm.to(d))
        _, z_want = oracle.pairmixer_layer(s, z_cur.cpu(), pm, state(layer))
        _check(f"pairmixer_module layer {i}", z_next, z_want, pm)
        z_cur = z_next
    assert torch.equal(z_got, z_cur)
    _, z_e2e = oracle.pairmixer_module(s, z, pm, state(mod), blocks)
    _e2e("pairmixer_module z", z_got, z_e2e, pm, blocks)


def test_pairmixer_msa_module_is_embed_then_layers(gpu_device):
    """MSA module = the input embedding (fp32, ~2^-15 relative) then the MSA layers in order (bit for bit);
    each layer on the GPU's own z and m within the bf16 bound of the oracle layer; end to end."""
    B, R, T, n_pad, E, blocks = 1, 16, 48, 5, 455, 2
    d = gpu_device
    torch.manual_seed(0)
    mod = init_module(PairMixerMSAModuleHip(384, 64, 128, E, blocks, 0.15, 0.25, use_paired_feature=True), 0)
    mod = mod.to(d).eval()
    g = torch.Generator().manual_seed(4)
    f, fd = _feats(B, R, T, n_pad, g, d)
    emb = torch.randn(B, T, E, generator=g)
    z = _randn((B, T, T, 128), g)
    pm = oracle.pair_mask_from_token_mask(f["token_pad_mask"])
    _, z_got = mod(None, z.to(d), emb.to(d), fd["msa"], fd["msa_mask"], fd["has_deletion"], fd["deletion_value"],
                   fd["msa_paired"], fd["token_pad_mask"])
    m_hi, m_tail = mod.embed(emb.to(d), fd["msa"], fd["has_deletion"], fd["deletion_value"], fd["msa_paired"])
    m_want = oracle.msa_embed(f["msa"], f["has_deletion"], f["deletion_value"], f["msa_paired"], emb, state(mod))
    torch.testing.assert_close(join_stream(m_hi, m_tail).cpu(), m_want, rtol=1e-4, atol=1e-5)
    z_hi, z_tail = split_stream(z.to(d))
    for i, layer in enumerate(mod.layers):
        z_in, m_in = join_stream(z_hi, z_tail).cpu(), join_stream(m_hi, m_tail).cpu()
        layer.forward_(None, z_hi, m_hi, pm.to(d), fd["msa_mask"], False, z_tail, m_tail)
        _, z_w, m_w = oracle.pairmixer_msa_layer(None, z_in, m_in, pm, f["msa_mask"], state(layer))
        _check(f"msa_module layer {i} z", join_stream(z_hi, z_tail), z_w, pm)
        _check(f"msa_module layer {i} m", join_stream(m_hi, m_tail), m_w, f["msa_mask"])
    assert torch.equal(z_got, join_stream(z_hi, z_tail))
    z_e2e = oracle.pairmixer_msa_module(z, emb, f, f["token_pad_mask"], state(mod), blocks)
    _e2e("pairmixer_msa_module z", z_got, z_e2e, pm, blocks)


@pytest.mark.parametrize("recycles", [0, 1])
def test_pairmixer_trunk_matches_oracle(gpu_device, recycles):
    """The recycling loop end to end (one MSA layer, one PairMixer layer per pass) against the oracle trunk;
    its parts are held to the bound alone above (recycling updates, MSA module layers, PairMixer layers)."""
    B, R, T, n_pad, E = 1, 8, 40, 4, 455
    torch.manual_seed(0)
    mod = init_module(PairMixerTrunkHip(384, 128, E, msa_blocks=1, num_blocks=1), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(5)
    f, fd = _feats(B, R, T, n_pad, g, gpu_device)
    s_init, z_init = _randn((B, T, 384), g), _randn((B, T, T, 128), g)
    emb = torch.randn(B, T, E, generator=g)
    s_got, z_got = mod(s_init.to(gpu_device), z_init.to(gpu_device), emb.to(gpu_device), fd, recycles)
    assert s_got.dtype == torch.float32 and z_got.dtype == torch.float32
    s_want, z_want = oracle.pairmixer_trunk(s_init, z_init, emb, f, state(mod), 1, 1, recycles)
    tok = f["token_pad_mask"]
    layers = 2 * (recycles + 1)
    _e2e(f"trunk recycles={recycles} z", z_got, z_want, oracle.pair_mask_from_token_mask(tok), layers)
    _e2e(f"trunk recycles={recycles} s", s_got, s_want, tok, 1)


@pytest.mark.parametrize("bf16_exact", [True, False])
def test_trunk_unconditional_branch_matches_oracle(gpu_device, bf16_exact):
    """z = z_init + uncond_transition(z_norm(z_init)) and s = s_init (pairmixer.py:266-273) against the oracle;
    the recycling loop does not run.  z_init is bf16-representable or a general fp32 stream (its LayerNorm then
    reads the bf16 part of the stream)."""
    B, T, d = 2, 50, gpu_device
    print(f"trunk uncond: B={B} T={T} bf16_exact={bf16_exact}", flush=True)
    torch.manual_seed(0)
    mod = init_module(PairMixerTrunkHip(384, 128, 455, msa_blocks=0, num_blocks=0, use_unconditional_branch=True), 0)
    mod = mod.to(d).eval()
    g = torch.Generator().manual_seed(6)
    s_init = _randn((B, T, 384), g)
    z_init = _randn((B, T, T, 128), g, 2.0) if bf16_exact else torch.randn(B, T, T, 128, generator=g) * 2.0
    s_got, z_got = mod(s_init.to(d), z_init.to(d), None, {}, unconditional=True)
    assert torch.equal(s_got.cpu(), s_init)
    assert z_got.dtype == torch.float32
    _, z_want = oracle.pairmixer_uncond(s_init, z_init, state(mod))
    _check(f"trunk uncond z (bf16_exact={bf16_exact})", z_got, z_want)
    if bf16_exact:
        with torch.no_grad():
            mod.uncond_transition.fc3.weight.zero_()
        _, z_zero = mod(s_init.to(d), z_init.to(d), None, {}, unconditional=True)
        assert torch.equal(z_zero.cpu(), z_init)   # a zero transition output leaves z_init bit for bit


def test_trunk_unconditional_requires_branch(gpu_device):
    mod = PairMixerTrunkHip(384, 128, 455, msa_blocks=0, num_blocks=0).to(gpu_device)
    with pytest.raises(ValueError, match="use_unconditional_branch=True"):
        mod(torch.zeros(1, 4, 384, device=gpu_device), torch.zeros(1, 4, 4, 128, device=gpu_device), None, {},
            unconditional=True)


def test_trunk_rejects_negative_recycles(gpu_device):
    mod = PairMixerTrunkHip(384, 128, 455, msa_blocks=1, num_blocks=1).to(gpu_device)
    with pytest.raises(ValueError, match="non-negative"):
        mod(None, None, None, {}, -1)


def test_trunk_ragged_batch_equals_systems_alone(gpu_device):
    """The reference's test_pairmixer_padding_integration at the trunk level: a ragged batch (the short system
    padded to the long one's token and MSA-row counts, padded entries random) gives each system's valid single and
    pair outputs bit-identical to running it alone, through the MSA input embedding, the MSA module, the PairMixer
    layers and a recycling pass."""
    E = 455
    torch.manual_seed(0)
    mod = init_module(PairMixerTrunkHip(384, 128, E, msa_blocks=1, num_blocks=2), 0).to(gpu_device).eval()
    g = torch.Generator().manual_seed(9)
    sizes = [(21, 5), (44, 8)]   # (tokens, MSA rows)
    T, R = 44, 8
    f, _ = _feats(2, R, T, 0, g, "cpu")
    s_init, z_init = _randn((2, T, 384), g), _randn((2, T, T, 128), g)
    emb = torch.randn(2, T, E, generator=g)
    tok = torch.zeros(2, T, dtype=torch.bool)
    msa_mask = torch.zeros(2, R, T, dtype=torch.bool)
    for b, (n, r) in enumerate(sizes):
        tok[b, :n] = True
        msa_mask[b, :r, :n] = f["msa_mask"][b, :r, :n]
    f["token_pad_mask"], f["msa_mask"] = tok, msa_mask
    dev = gpu_device
    fd = {k: v.to(dev) for k, v in f.items()}
    s_rag, z_rag = mod(s_init.to(dev), z_init.to(dev), emb.to(dev), fd, 1)
    for b, (n, r) in enumerate(sizes):
        fb = {k: v[b:b + 1, :r, :n].contiguous().to(dev) if v.ndim >= 3 else v[b:b + 1, :n].contiguous().to(dev)
              for k, v in f.items()}
        s_one, z_one = mod(s_init[b:b + 1, :n].contiguous().to(dev), z_init[b:b + 1, :n, :n].contiguous().to(dev),
                           emb[b:b + 1, :n].contiguous().to(dev), fb, 1)
        ds = (s_rag[b, :n] - s_one[0]).abs().max().item()
        dz = (z_rag[b, :n, :n] - z_one[0]).abs().max().item()
        print(f"system {b} (n={n}, S={r}): max |ragged - alone| s={ds:.3e} z={dz:.3e}", flush=True)
        assert ds == 0.0 and dz == 0.0
