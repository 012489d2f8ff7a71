"""CPU oracle for the moe-stream expert hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` may use it, and only as the checker.

Modules:
  numerics   -- numpy restatement of the MLX arithmetic on the path
                (affine 4-bit dequant, gather_qmm, both SwiGLUs, both routing
                rules, lookahead top-k, weighted combine, whole MoE blocks).
  policy     -- pure-Python restatement of ``ExpertPool``'s slot bookkeeping
                (``_alloc``/``_touch``/``prefetch``/``acquire``/``stats``).
  layout     -- expert record layout of the repacked store.
  synth      -- seeded synthetic inputs for the five benchmark workloads.

Parity status per function is listed in each module header.
"""
