"""Gated DeltaNet core on the HIP kernels, for a whole batch at once.

Drop-in for the device work of ``GatedDeltaNet._forward_prefill`` /
``_forward_decode`` (layers/gated_delta_net.py:178-270) between the
projections and ``out_proj``, which the reference runs once per sequence
(models/qwen3_5.py:215-240):

    mixed = silu(causal_conv1d(in_proj_qkv(x)))      -> nq_gdn_conv1d
    q, k, v = split(mixed)
    y = delta_rule(q, k, v, a, b, A_log, dt_bias)    -> nq_gdn_prefill / nq_gdn_decode
    y = RMSNormGated(y, z)                           -> nq_gated_rmsnorm

``layer`` is the reference's module; only its parameters, buffers and state
pools are read (``conv1d.weight``, ``A_log``, ``dt_bias``, ``norm.weight``,
``norm.eps``, ``conv_states``, ``recurrent_states`` -- the recurrent pool in
float32).  Prefill starts every sequence from zero states, as the reference
does, and leaves each sequence's final conv and recurrent state in its slot.
"""
from __future__ import annotations

import torch

from .. import kernels


def gdn_core(layer, qkv_raw: torch.Tensor, z: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
             state_indices: torch.Tensor, cu_seqlens: torch.Tensor | None = None) -> torch.Tensor:
    """``qkv_raw [T, conv_dim]`` (``in_proj_qkv`` output), ``z [T, value_dim]``,
    ``a, b [T, HV]``; ``state_indices [N]`` int32 (decode: N = T, one token
    per sequence; prefill: ``cu_seqlens [N + 1]`` int32 packs the sequences).
    Returns the normalized output ``[T, value_dim]`` (the ``out_proj`` input).
    """
    T = qkv_raw.shape[0]
    H, HV = layer.num_k_heads, layer.num_v_heads
    Dk, Dv = layer.head_k_dim, layer.head_v_dim
    kd, vd = H * Dk, HV * Dv
    w = layer.conv1d.weight.detach().reshape(qkv_raw.shape[1], -1).to(qkv_raw.dtype).contiguous()
    mixed = kernels.gdn_conv1d(qkv_raw, w, layer.conv_states, state_indices, cu_seqlens=cu_seqlens)
    q = mixed[:, :kd].view(T, H, Dk)
    k = mixed[:, kd:2 * kd].view(T, H, Dk)
    v = mixed[:, 2 * kd:].view(T, HV, Dv)
    A_log = layer.A_log.detach().float()
    dt_bias = layer.dt_bias.detach().float()
    if cu_seqlens is None:
        y = kernels.gdn_decode(q, k, v, a, b, A_log, dt_bias, layer.recurrent_states, state_indices)
    else:
        y = kernels.gdn_prefill(q, k, v, a, b, A_log, dt_bias, cu_seqlens, layer.recurrent_states, state_indices)
    out = y.view(T, vd)
    kernels.gated_rmsnorm(out.view(-1, Dv), z.reshape(-1, Dv), layer.norm.weight.detach().float().contiguous(),
                          layer.norm.eps, out=out.view(-1, Dv))
    return out
