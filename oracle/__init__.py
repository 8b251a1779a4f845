"""CPU oracle for the masked flash-attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``tagseq2tagseq_amd``)
imports, links or executes anything under ``oracle/``.  The only permitted
callers are ``tests/``, ``__graft_entry__.smoke()`` (as the checker) and the
``cpu_baseline`` leg of ``bench.py``.

Contents
--------
``mask_oracle``   restatement of the reference's mask semantics
                  (document ids, grant bitmasks, ``mask_mod``) and of
                  torch's BlockMask tile classification / ordered index lists.
``attn_oracle``   dense float64 masked attention forward and backward, the
                  arithmetic of torch's eager ``math_attention`` /
                  ``sdpa_dense_backward`` that the reference calls.
``tile_oracle``   ctypes wrapper over ``tile_oracle.c``: brute-force per-tile
                  pair counts for full-size (T = 16k / 32k) classification checks.

Every function cites the reference (or torch) file:line it restates.  Paths
without a prefix are relative to the reference repository root; ``torch/``
means the installed PyTorch 2.10.0 package.
"""
