"""ORACLE — TEST INFRASTRUCTURE ONLY.

CPU restatement of BatchSpec's speculative-verification path, used as the checker
of the gfx950 kernels.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``batchspec_amd``) never does and has no CPU fallback.

Modules (each function cites the reference file:line it follows):
  attention  paged gather + masked softmax attention in fp32 (numpy)
  append     paged KV append scatter (numpy)
  paging     CSR page-table allocator / insert / delete (numpy)
  masks      MTP interleaved mask and draft-tree ancestor words (numpy)
  accept     greedy acceptance (numpy) and the canonical stochastic acceptance
             (C, accept.c, via ctypes)

How each function is pinned (tests/test_oracle_*.py):
  attention  torch scaled_dot_product_attention on the gathered pages, pure-Python
             loops on tiny inputs, page-permutation / GQA / chain-tree / decode
             invariances, sink+window view == attention over the compacted cache
  append     gather(append(x)) == x, untouched slots unchanged, explicit loops
  paging     the known-answer examples of batchspec/backends/utils/paging.py:89-129
  masks      the k=2 known answer of batchspec/backends/mtp_engine.py:360-368
  accept     greedy: numpy.argmax + exhaustive brute force on tiny vocabularies;
             stochastic: exp2 vs libm within 3 ulp, softmax vs float64, the
             tree draw vs a float64 linear inverse-CDF scan, q == p accepts all,
             disjoint supports reject at 0, and a chi-square test that the emitted
             token is distributed as p (speculative-sampling invariant).
  The exact rounding order of FlashInfer's own sampling kernels (internal RNG) is
  not reproducible: that part is parity unpinned; the canonical order above is the
  contract instead.
"""
