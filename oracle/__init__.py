"""Oracle for the FlexAttention hot path — TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms on the CPU so that the
MI355X kernels can be checked against them.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
it, and only as the checker / the timed CPU baseline.  The product package
(``pallas_flexattn``) never imports anything from here.

Contents and what pins each function (a function with no independent check
would be marked "parity unpinned"; none is):

* ``masks``       — mask predicates restated from ``src/pallas_flexattn/mask_mod.py:15-43``
                    (+ the document predicate the reference leaves as a stub,
                    ``mask_mod.py:46-59``).  Pinned by closed forms in the tests.
* ``block_mask_ref`` — pure-Python restatement of the 3x3 sampling rule of
                    ``block_mask.py:54-129`` and the closed forms of
                    ``block_mask.py:132-218``.  Pinned by the reference's own
                    test assertions (``tests/test_block_mask.py``) and closed forms.
* ``attention``   — float64 materialised attention restating
                    ``flash_attn.py:33-56`` (``mha_reference``), extended with
                    score mods and GQA, plus its analytic backward.  Pinned by
                    finite differences, softmax invariants, GQA == repeat_kv,
                    and the C tiled restatement.
* ``tiled``       — ctypes front end of ``tiled_ref.c``: a C/OpenMP restatement
                    of the reference's tiled Pallas kernels (fwd ``flash_attn.py:59-108``,
                    bwd ``:168-407``) with the same bf16 cast points.  Used as the CPU
                    baseline and cross-checked against ``attention``.
* ``bf16``        — float32 -> bfloat16 round-to-nearest-even in numpy.
* ``fp8``         — OCP e4m3 codec, the fp8 path's block quantisation and a
                    model of its P rounding (no reference counterpart: the
                    reference has no fp8 path).  Pinned against torch's
                    float8_e4m3fn conversion, closed forms, the quantisation's
                    defining invariants and ``attention``.
"""
