"""CPU oracle for the wmma_ops hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import, call, link or execute anything under ``oracle/``, and only as the checker or
the reported CPU baseline.  The product (``wmma_ops_amd``) never routes through it.

Modules
  gemm       FP16 GEMM + alpha/beta epilogue + split-K partition
             (reference: wmma_gemm.hip:636-666, 1891-1994; wmma_xor_swizzle.hpp:293-353;
             known-answer test test_fragment_loading.py:225-274)
  int4       GPTQ int4 pack/unpack, this library's prepacked layout, dequantisation and
             the W4A16 product (no reference code exists; semantics from the task's
             W4A16 definition)
  attention  scaled-dot-product attention (reference API: README.md:221-251)
  cref       ctypes binding of the plain-C restatement in gemm_ref.c / int4_ref.c

Pinning (what each function is checked against, in tests/test_oracle.py):
  gemm.gemm_ref          known-answer test; float64 brute force; identity / zero /
                         permutation / linearity invariants; the C restatement
  gemm.splitk_partition  restated from wmma_xor_swizzle.hpp:293-332; sum over splits
                         equals the unsplit product
  int4.*                 round trips, bijection (nibble multiset), independent C
                         restatement, fp16 rounding via two independent routes,
                         special cases (q == z -> 0, s = 1 & z = 0 -> integers).
                         The reference holds no INT4 vectors, so parity with the
                         reference itself is unpinned; the layout is pinned to this
                         library's written specification.
  attention.sdpa_ref     float64 naive softmax; identical-V-rows, causal row 0, scale 0
                         (uniform / prefix mean) and key-permutation invariants
"""
