"""CPU oracle for the decoder-layer monokernel path: TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's decode-layer
monokernel (yuychang/sgl-amd-mono, ``sgl_amd_mono/glm53/gfx950/kernel.py`` and the
FP4 indexer / MXFP4 expert code it shares with ``deepseek_v4``, ``deepseek_v41`` and
``minimax_m31``). Every function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline. The
product path (``sgl_amd_mono_amd``) never imports it and has no CPU fallback.

Pinning: each public function here is checked in ``tests/test_oracle_*.py`` against
an independent fact: exhaustive code tables (FP8 / E2M1 / E8M0), textbook closed
forms in float64 (RMSNorm, RoPE, Hadamard, softmax), brute-force stable sorts for
the top-k rules, an fp64 dense restatement for the scores and attention, and the
committed golden vectors under ``tests/golden/``. Functions without such a check are
marked "parity unpinned" in their docstring.
"""
