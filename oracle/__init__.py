"""CPU oracle for the Pairformer hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``bioemu2_amd``) never routes through it and
fails loudly when its HIP library is missing.

Every function is a float32 PyTorch-on-CPU restatement of the reference's
algorithm (itsawesomeabhishek/bioemu2) and cites the reference file:line it
follows.  Parameters are passed as dicts whose keys are the reference modules'
``state_dict`` keys, so ``oracle.trimul(x, mask, module.state_dict(), ...)``
works for both the reference classes and the drop-in HIP classes.

How each function is pinned (see ``tests/test_oracle_*.py``):

* ``trimul``      — brute-force Python loops (tiny N), the
                    incoming(x) == outgoing(x^T, a<->b swapped)^T identity, the
                    bit-exact masking and padding invariances of the reference
                    tests (test_triangle_multiplication.py:303-399).
* ``triangle_attention`` — NOT in the reference (AF3 suppl. Alg. 14/15).
                    Pinned by brute-force loops, ending(z) == starting(z^T)^T,
                    reduction to per-row SDPA with a zero bias, and the
                    fully-masked-row closed form (uniform weights).
* ``attention_pair_bias`` — brute-force loops, reduction to torch SDPA with an
                    additive mask, tiled == untiled, multiplicity == separate runs,
                    bitwise padding invariance (test_attention_pair_bias.py:805-867).
* ``attention_pair_bias_sliding_window`` — brute-force loops over absolute
                    atom positions, a planted one-hot bias that must select the
                    key the centred window puts at that offset (the window's
                    own queries sit at offsets ctx..ctx+W-1), reduction to
                    ``attention_pair_bias`` per window when H == W, sequence-edge
                    keys masked, multiplicity == separate runs.
* ``distogram``   — brute-force loops; the output is exactly symmetric in
                    (i, j); a planted variant without the transpose fails it.
* ``pairwise_conditioning`` — brute-force loops; the concatenation order
                    (z_trunk first) is pinned by an asymmetric LayerNorm; zero
                    transitions reduce it to LN + projection.
* ``outer_product_mean`` — brute-force loops over S, masked rows contribute
                    exact zeros (test_outer_product_mean.py:286-310), the
                    divisor is the per-batch valid-row count (duplicating the
                    MSA leaves the mean unchanged).
* ``pair_weighted_averaging`` — brute-force loops, the all-masked row (uniform
                    average over the N keys), a single valid key (o = v of that
                    key exactly), MSA-row independence of the weights.
* ``transition``  — brute-force loops and the SwiGLU closed form.
* ``pairformer_block`` (AF3 suppl. Alg. 17), ``pairmixer_layer``
  (pairmixer.py:430-456) and ``pairmixer_msa_layer`` (pairmixer.py:711-757)
                  — compositions of the pinned terms above, pinned in
                    tests/test_oracle_compositions.py: with every output
                    projection zeroed they return their inputs bit for bit;
                    with one left non-zero they return input + that op's
                    update (computed from the op function and a sub-dict the
                    test builds itself); with two consecutive ops non-zero
                    the second sees the first one's output, and the reversed
                    order (a negative control) differs.

No function here is "parity unpinned".
"""

from .pairformer_ref import (  # noqa: F401
    attention_pair_bias,
    attention_pair_bias_sliding_window,
    distogram,
    ln_linear,
    msa_embed,
    outer_product_mean,
    pair_mask_from_token_mask,
    pair_weighted_averaging,
    pairformer_block,
    pairmixer_layer,
    pairmixer_module,
    pairmixer_msa_layer,
    pairmixer_msa_module,
    pairmixer_trunk,
    pairmixer_uncond,
    pairwise_conditioning,
    sliding_window_keys,
    transition,
    triangle_attention,
    trimul,
)
