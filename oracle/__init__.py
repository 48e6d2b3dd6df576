"""CPU oracle for nano_qwen's paged attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on its paged
attention path, so that the HIP kernels in ``nano_qwen_amd`` can be checked
against it.  It is a checker, never a product path: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  ``nano_qwen_amd`` never imports it and has no CPU fallback.

Modules
-------
``fp8``        OCP float8-e4m3fn encode/decode with round-to-nearest-even
               (numpy integer/float arithmetic).
``paged``      ``store_kvcache`` scatter, paged decode attention and causal
               varlen prefill attention in float64 (numpy).
``metadata``   closed forms of ``ModelRunner.prepare_prefill`` /
               ``prepare_decode`` / ``_prepare_decode_kernel``.
``inputs``     seeded synthetic inputs for the five benchmark configurations.
``sdpa_path``  the CPU baseline: torch block gather + repeat_interleave +
               ``scaled_dot_product_attention`` (the path ``bench.py`` times
               on the host cores).
``qk_norm_rope`` q/k Gemma RMS norm + partial rotary embedding + KV store
               (float32 operations in the reference's rounding order).
``output_gate`` the ``attn_output * sigmoid(gate)`` gate of Qwen3.5.
``gdn``        the gated delta rule (decode step, packed prefill) in float64
               and the gated RMS norm of its output.

Parity pinning (what checks each function; see ``tests/test_oracle.py``):

* ``paged.store_kvcache``  -- closed form (flat-row assignment) and the
  bit-level round trip; no floating point involved.
* ``fp8.encode_e4m3fn``    -- exhaustively against torch's
  ``float8_e4m3fn`` cast (a library routine) and all 256 codes round-trip.
* ``paged.paged_decode`` / ``paged.varlen_prefill`` -- against torch
  ``scaled_dot_product_attention`` in float64 on contiguous inputs, a
  pure-Python brute force on tiny inputs, closed-form special cases
  (ctx = 1 gives ``v[0]``; q = 0 gives the mean of V; a dominant score selects
  one row) and invariants (physical block permutation, decode == last row of
  the causal prefill, padding of block tables).
* ``metadata``             -- restated closed forms, checked against a
  token-by-token simulation of the reference's block bookkeeping.

Each of the later modules states in its docstring what pins it; the tests
are ``tests/test_oracle_qk_norm_rope.py`` and ``tests/test_oracle_gdn.py``.

flash_attn's own bit-level rounding (the third-party library the reference
calls, unpinned version, not installed here) is NOT pinned: the attention
oracle is exact float64 softmax attention, and the kernels are held to the
tolerance stated in the tests.
"""
