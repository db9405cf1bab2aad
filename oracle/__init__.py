"""CPU oracle for the selective-scan hot path.

TEST INFRASTRUCTURE ONLY. Nothing in ``selectssm_amd`` imports this package.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import, call, link or run anything under ``oracle/``, and only as the
checker or the timed CPU baseline, never as the product path.

Modules:
  ssm_oracle   numpy restatement (fp64 closed form + fp32 restatements of the
               reference's chunked / recursive / custom-VJP algorithms).
  ssm_oracle.c C restatement of the reference's custom-VJP path (recursive
               forward + recursive adjoint backward), OpenMP over rows; built
               into ``oracle/libssm_oracle.so`` by ``oracle/Makefile``.
"""
