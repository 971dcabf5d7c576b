"""CPU oracle for the DeepSeeker MoE-layer forward -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU (numpy integer/byte work, torch fp32
GEMMs), what the reference's MoE layer computes, so that the HIP library can
be checked against it on identical inputs.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to compare against or as the timed CPU baseline.  The product
path (``dsk_moe``) never imports it and never falls back to it.

Modules and the reference code each one follows (paths relative to the
reference repository):

* ``formats``  -- FP4 e2m1 / E8M0 decode (``src/deepseeker/metal_fp4.py:21-26,
  96-103, 122-168``; ``src/deepseeker/mlx_weights.py:66-79, 148-166``), the
  FP4 quantiser defined by the workload spec, and the q3 affine format
  (``src/deepseeker/mlx_weights.py:119-145``;
  ``scripts/requant_experts_3bit.py:69-83``) in this build's canonical
  bit layout.
* ``router``   -- gate logits, sigmoid / sqrt-softplus scores, biased top-k and
  normalised weights (``src/deepseeker/mlx_forward.py:62-81``;
  ``tests/test_mlx_numerics.py:69-89``).
* ``dispatch`` -- token->expert grouping (``src/deepseeker/mlx_forward.py:294-312,
  388-396``; ``src/deepseeker/moe_align.py:21-46``;
  ``src/deepseeker/grouped.py:19-31``).
* ``layer``    -- expert SwiGLU, combine and shared expert
  (``src/deepseeker/mlx_forward.py:257-419``;
  ``src/deepseeker/mlx_runner.py:765-783``).
* ``synth``    -- seeded synthetic layers for the five workload configurations.

Parity status of each function is stated in its docstring ("pinned by ..." or
"parity unpinned").
"""
