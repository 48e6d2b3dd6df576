"""Qwen3.5's attention output gate, restated in numpy.

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker for the
gated decode store and ``nq_output_gate``.

Reference, models/qwen3_5.py:140-142 (eager, not compiled)::

    attn_output = attn_output.reshape(-1, self.q_size)
    gate = gate.reshape(-1, self.q_size)
    attn_output = attn_output * torch.sigmoid(gate)

On 16-bit tensors eager torch computes ``sigmoid`` in float32 and rounds it
to the dtype, then multiplies two dtype values in float32 (exact for 16-bit
significands) and rounds the product once.  ``attn_output`` is the attention
result already rounded to the dtype.
"""
from __future__ import annotations

import numpy as np

from .qk_norm_rope import round_to

F32 = np.float32


def sigmoid32(g: np.ndarray) -> np.ndarray:
    """1 / (1 + exp(-g)) in float32 operations."""
    g = np.asarray(g, dtype=F32)
    with np.errstate(over="ignore"):
        e = np.exp(-g).astype(F32)
    return (F32(1.0) / (F32(1.0) + e)).astype(F32)


def output_gate(o: np.ndarray, gate: np.ndarray, dtype: str) -> np.ndarray:
    """rnd(rnd(o) * rnd(sigmoid(gate))) elementwise, rnd = round to ``dtype``."""
    s = round_to(sigmoid32(gate), dtype)
    return round_to(round_to(o, dtype) * s, dtype)
