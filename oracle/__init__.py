"""CPU oracle for the fused MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference's non-expert-parallel
``fused_moe`` computes (AdaMLLab/FlashFusedMoE, ``src/flashfusemoe``), so that
the HIP kernels in ``flashfusedmoe_amd`` can be checked against it on identical
seeded inputs.  It is the checker, never the thing measured or shipped:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it;
* ``flashfusedmoe_amd`` never imports it and has no CPU fallback.

Modules
-------
``routing``  numpy: max-tokens heuristic, top-k rule, stable permutation,
             capacity keep-mask, expand_to_batch.  Integer/index work is exact.
``fused``    torch-CPU restatement of ``_FusedMoEAutograd`` forward and the
             hand-written backward, on the reference's padded [E*mt, D] layout,
             with the reference's rounding points, plus the aux/z losses and
             metrics block of ``fused_moe()``.
``unfused``  torch-CPU restatement of the reference's unfused test oracle
             ``unfused_moe`` (per-slot, per-expert loop, autograd backward); it
             is also the CPU baseline timed by ``bench.py``.

How each function is pinned (the checks live in ``tests/test_oracle_*.py``):

* ``estimate_max_tokens``: the reference's own known answers
  (tests/test_production.py:37-47) plus the closed form at every config.
* ``topk_select``: brute force (lexicographic sort on (-value, index)) on
  tie-heavy small-integer inputs, and ``torch.topk`` on tie-free inputs.
* ``stable_permutation`` / ``expand_to_batch`` / ``capacity_keep``: numpy's
  stable argsort and the closed-form rank definition, by brute force.
* ``fused.forward``: the independent ``unfused`` restatement in fp64 (two
  different algorithms: padded batched layout vs per-expert masked loop).
* ``fused.backward``: ``torch.autograd`` through ``unfused`` in fp64 for all
  four gradients (hidden, gate, w_up, w_down); GLU derivatives against
  autograd of the GLU forward.
* aux/z losses: closed forms and autograd of ``torch.logsumexp``.

Parity unpinned: none of the functions above.  The bf16 bit patterns of the
reference's cuBLAS GEMM outputs cannot be pinned without an NVIDIA GPU; bf16
results are compared within a stated tolerance instead.
"""
