"""``rms_norm_gated`` (drop-in for the reference's ``python/logssms/kernel/norm.py:151-187``),
on the gfx950 kernel ``gdn_rms_norm_gated`` (``csrc/norm.hip``)."""

from __future__ import annotations

import torch

from .. import _lib


def rms_norm_gated(
    hidden_states: torch.Tensor,
    gate: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
) -> torch.Tensor:
    """Per row of ``hidden_states.shape[-1]`` channels:
    ``(x * rsqrt(mean(x^2) + eps)) * weight * silu(gate)``, computed in fp32 and
    returned in the dtype and shape of ``hidden_states``.  ``gate`` may be a
    strided view (the reference indexes it as ``gate.reshape(-1, gate.shape[-2], n)``)."""
    assert hidden_states.shape == gate.shape
    assert hidden_states.shape[-1] == weight.numel()
    assert hidden_states.is_cuda and gate.is_cuda and weight.is_cuda
    num_cols = hidden_states.shape[-1]
    hidden = hidden_states.reshape(-1, num_cols).contiguous()
    gate3 = gate.reshape(-1, gate.shape[-2], num_cols) if gate.ndim > 1 else gate.view(1, 1, num_cols)
    weight = weight.contiguous()
    output = torch.empty_like(hidden)
    _lib.call(
        "gdn_rms_norm_gated",
        hidden.data_ptr(), _lib.dtype_code(hidden.dtype), hidden.shape[0], num_cols,
        gate3.data_ptr(), _lib.dtype_code(gate3.dtype), gate3.shape[1], gate3.stride(0), gate3.stride(1),
        gate3.stride(2), weight.data_ptr(), _lib.dtype_code(weight.dtype), float(eps), output.data_ptr(),
        _lib.stream_of(hidden),
    )
    return output.view(hidden_states.shape)


__all__ = ["rms_norm_gated"]
