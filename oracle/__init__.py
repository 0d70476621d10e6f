"""CPU oracle for the hierarchical-mask flash-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``kerneldev_amd``)
imports, calls or links anything in this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, and only as the checker / the reported CPU baseline -- never as the thing
being measured or shipped.

Modules
-------
mask       -- the 7-term cocktail-party mask formula and its fallbacks
              (restates ``original_kernel.py:478-517`` and ``:512-517``).
tilemap    -- exhaustive full/partial/empty tile classification of a dense
              mask and the per-row-block work lists the kernels consume.
metadata   -- tokens -> (is_prefix, in_span, span_id) for both derivations
              the reference has (``data_builder.py:603-643`` and
              ``model.py:209-240``), written as plain per-token loops.
attention  -- dense masked attention forward/backward on the CPU
              (fp64 / fp32) with base-2 LSE and Delta, plus the eager SDPA
              baseline that follows ``original_kernel.py:2002-2032``.
hadamard   -- Sylvester Walsh-Hadamard transform with random signs.
fp8        -- OCP e4m3fn round-to-nearest-even quantisation, bit level.
span_head  -- the cocktail-party head's span pooling and scores
              (restates ``model.py:263-296``, Python loops kept).

Pinning: every function above is checked in ``tests/test_oracle_*.py``
against closed forms, hand-built truth tables, brute force on tiny inputs,
library routines (scipy's Hadamard, torch's float8 cast, torch SDPA) and
invariants.  The reference ships no golden vectors or tests of its own for
this path, so nothing here is checked against reference-produced vectors.
The Triton kernels' own rounding quirks (bf16-rounded scale constants,
tf32 dots, NaN rows, causal-truncated backward loops) are deliberately NOT
reproduced and stay "parity unpinned" by design.
"""
