"""CPU oracle for the moe-stream expert hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
package.  ``tests/`` and ``__graft_entry__.smoke()`` use it as the checker
(the GPU results are compared with it); the CPU-baseline leg of ``bench.py``
times ``cpu_block`` on the host cores as the reported CPU baseline (measured
beside the GPU, never as the GPU's result).

Modules:
  numerics   -- numpy restatement of the MLX arithmetic on the path
                (affine 4-bit dequant, gather_qmm, both SwiGLUs, both routing
                rules, lookahead top-k, weighted combine, whole MoE blocks).
  policy     -- pure-Python restatement of ``ExpertPool``'s slot bookkeeping
                (``_alloc``/``_touch``/``prefetch``/``acquire``/``stats``) and
                of the reference's prefetch-aware pool simulator.
  layout     -- expert record layout of the repacked store.
  cpu_block  -- torch-CPU restatement of the router + expert block, the
                timed CPU baseline of ``bench.py``.

The seeded synthetic inputs live in the product package
(``moe_stream_amd.synth``): they are workloads, not checks.

Parity status per function is listed in each module header.
"""
