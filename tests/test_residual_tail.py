"""The residual-tail format (CPU): the numpy statement in tests/_helpers.py against the mathematics.

value = hi + t * 2^(E(hi) - 142): hi is the nearest bf16, t counts 1/256ths of
hi's unit in the last place (|t| <= 127), so a round trip errs by at most one
tail unit (half a unit unless the remainder clamps at +-127): relative error
<= 2^-15, i.e. ~15-16 significant bits.
"""

from __future__ import annotations

import numpy as np
import torch

from tests._helpers import np_bf16_rne, np_bf16_to_f32, np_tail_decode, np_tail_encode


def _samples(n=200_000, seed=0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, n))).astype(np.float32)
    return np.concatenate([x, np.array([0.0, -0.0, 1.0, -1.0, 3.0, 1.0 - 2 ** -24, 2.0 ** -100, 65504.0],
                                       dtype=np.float32)])


def test_bf16_rounding_matches_torch():
    x = _samples()
    assert np.array_equal(np_bf16_rne(x), torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy()
                          .view(np.uint16))


def test_round_trip_keeps_15_bits():
    x = _samples()
    hi, t = np_tail_encode(x)
    y = np_tail_decode(hi, t)
    assert np.all(np.abs(t.astype(np.int32)) <= 127)
    err = np.abs(y.astype(np.float64) - x.astype(np.float64))
    unit = np.ldexp(1.0, ((hi >> 7) & 0xFF).astype(np.int32) - 142)
    # half a tail unit except where the remainder clamps at +-127: then at most one unit
    assert np.all(err <= np.where(np.abs(t.astype(np.int32)) == 127, 1.0, 0.5) * unit * (1 + 1e-6))
    # one unit = ulp(hi) / 256 <= |x| * 2^-15 (hi normal)
    assert np.all(err <= np.abs(x.astype(np.float64)) * 2.0 ** -15 + 1e-38)
    # the value part alone is the nearest bf16 (so readers of hi see the round-to-nearest stream)
    assert np.array_equal(hi, np_bf16_rne(x))


def test_tail_is_zero_for_bf16_values():
    x = np_bf16_to_f32(np_bf16_rne(_samples()))
    _, t = np_tail_encode(x)
    assert np.all(t == 0)


def test_negative_control_ulp_scale():
    """A tail unit one binade off (2^(E-141)) breaks the 15-bit bound: the exponent offset is pinned."""
    x = _samples(20_000, seed=1)
    hi, t = np_tail_encode(x)
    e = ((hi >> 7) & 0xFF).astype(np.int32)
    wrong = np_bf16_to_f32(hi).astype(np.float64) + np.ldexp(t.astype(np.float64), e - 141)
    err = np.abs(wrong - x.astype(np.float64))
    assert np.any(err > np.abs(x.astype(np.float64)) * 2.0 ** -15 + 1e-38)


def test_bf16_of_joined_value_is_hi():
    """Rounding a stream's value hi + tail to bf16 gives hi back bit for bit (|tail| <= 127/256 ulp, and at a
    binade edge the nearest-even tie keeps hi), so a bf16 join may return hi without a pass over the stream."""
    x = _samples()
    hi, t = np_tail_encode(x)
    back = np_bf16_rne(np_tail_decode(hi, t))
    # the one difference: -0 + 0 is +0 in the fp32 join, while hi keeps the zero's sign
    assert np.array_equal(np.where(hi == 0x8000, 0, back), np.where(hi == 0x8000, 0, hi))
    assert np.all(back[hi == 0x8000] == 0)
    # values within one bf16 ulp of binade edges (where the spacing halves below the edge), every fp32
    # step of the last 2^9 on either side
    edges = np.ldexp(1.0, np.arange(-20, 21)).astype(np.float64)
    steps = np.arange(-512, 513, dtype=np.float64)
    near = np.concatenate([(e + steps * e * 2.0 ** -24) for e in edges]).astype(np.float32)
    near = np.concatenate([near, -near])
    hn, tn = np_tail_encode(near)
    assert np.array_equal(np_bf16_rne(np_tail_decode(hn, tn)), hn)
    assert np.array_equal(hn, np_bf16_rne(near))

