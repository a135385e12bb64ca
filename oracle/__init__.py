"""CPU oracle for the blockwise-causal attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, in the
bench, as the timed CPU baseline). The product package ``dexter_amd`` never
imports it and has no CPU fallback.

Contents (each function cites the reference file:line it restates; paths are
under ``python/dexter/`` of raikonenfnu/dexter-labs):

* ``attention``  torch fp32 restatement of the reference attention op
                 (``ops/reference/attention.py:22-77``): mask + masked softmax.
* ``rope``       torch restatement of the reference QK-norm + rotary
                 (``ops/reference/rope.py:10-56``), with its intermediate
                 rounding to the input dtype.
* ``kv_cache``   the KV-cache append/commit contract (``models/dreamzero/model.py:35-65``).
* ``norm``       torch restatement of the reference adaLN modulation and gated
                 residual (``ops/reference/norm.py:16-25``), with the reference's
                 per-op rounding, plus the single-rounding forms the fused
                 kernels compute.
* ``brute``      fp64 brute force (numpy, explicit loops) of attention, the
                 prologue and the adaLN/gated-residual pair, written
                 independently of the torch restatements;
                 the tests pin the restatements against it, against
                 ``torch.nn.functional.scaled_dot_product_attention`` and
                 against closed forms.

Pinning status: every function here is pinned (tests/test_oracle.py); none is
"parity unpinned". The reference ships no golden vectors for this path, so
the pins are the fp64 brute force, a library routine and closed-form cases.
"""
