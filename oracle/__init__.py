"""CPU oracle for the quantized-weight matrix path -- TEST INFRASTRUCTURE ONLY.

This package is a plain numpy restatement of the reference's algorithms for the
MXFP4 / FP8 matrix path (codecs, A16 and A8 linears, FP8 block GEMM, routing,
expert sort, tile list, MoE layer, DSA indexer + top-k, sparse MLA decode).
Each function cites the reference file:line it restates (paths relative to the
reference repository root).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only as the checker.  The product package ``mosaic_amd``
never imports it: the product path runs the HIP kernels or raises.

Pinning (how each function is checked by something other than itself) is
listed per module docstring; ``tests/test_oracle_*.py`` hold those checks.
"""
