"""CPU oracle for the Qwen3-4B greedy-decode hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``thing-htn-2026_amd/``)
imports, links or runs anything from this package. It is used by ``tests/``
as the checker, by ``__graft_entry__.smoke()`` to check one small GPU call,
and by ``bench.py``'s ``cpu_baseline`` leg as the timed CPU restatement.

Modules
-------
``ref_torch``  torch-CPU restatement of the reference's per-op formulas and
               of one whole decode / prefill step (the primary oracle). Each
               function cites the reference file:line it restates.
``ref_numpy``  an independent numpy restatement with a hand-written bf16
               round-to-nearest-even, used to cross-check ``ref_torch``.
``weights``    the counter-based random-init weight generator (integer-only
               arithmetic, so every platform produces the same bits).
``model``      ``CpuQwen3``: weights + static KV cache + the reference's
               generate() protocol on the CPU, built from ``ref_torch``.

Pinning (what each function is checked against) is listed in the tests that
exercise it: ``tests/test_oracle_hf.py`` (bit-exact against the Transformers
Qwen3 modules on CPU, the module the reference's own twin tests compare to),
``tests/test_oracle_invariants.py`` (closed forms, brute force in float64,
invariants the reference's tests state) and ``tests/test_oracle_model.py``
(whole-model greedy decode against ``transformers.Qwen3ForCausalLM``).
"""
