"""CPU oracle for the SD1.5 UNet hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the timed CPU reference).  The product path never routes through it.

Modules:
  weights   parameter inventory of the reference's UNet graph and the seeded generator
  unet_ref  fp32 torch restatement of the reference engine's ops, blocks and graph
  lcm       closed-form time projection, LCM scheduler and CFG combine
"""
