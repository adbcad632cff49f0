"""``prepare_gdn`` (drop-in for the reference's
``python/logssms/kernel/fused.py:120-158``)."""

from __future__ import annotations

import torch

from .. import _lib


def prepare_gdn(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    beta: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """fused.py:120-158: ``q, k <- x rsqrt(sum x^2 + 1e-6)`` per head (stored in
    the input dtype), ``v`` copied exactly, ``g = -exp(A_log) softplus(gate +
    dt_bias)`` (threshold 20) and ``beta = sigmoid(beta)`` in fp32.  Inputs may
    be strided views; outputs are contiguous."""
    assert query.is_cuda and query.ndim == key.ndim == value.ndim == 4
    batch_size, tokens, key_heads, key_dim = query.shape
    value_heads, value_dim = value.shape[2:]
    assert key.shape == query.shape and value.shape[:2] == query.shape[:2]
    assert key_heads > 0 and value_heads % key_heads == 0
    assert gate.shape == beta.shape == (batch_size, tokens, value_heads)
    assert A_log.shape == dt_bias.shape == (value_heads,)
    assert query.dtype in (torch.float16, torch.bfloat16, torch.float32)
    for tensor in (key, value):
        assert tensor.dtype == query.dtype and tensor.device == query.device
    for tensor in (gate, beta, A_log, dt_bias):
        assert tensor.device == query.device
        assert tensor.dtype in (torch.float16, torch.bfloat16, torch.float32)
    q_out = torch.empty(query.shape, device=query.device, dtype=query.dtype)
    k_out = torch.empty_like(q_out)
    v_out = torch.empty(value.shape, device=value.device, dtype=value.dtype)
    gate_out = torch.empty(gate.shape, device=gate.device, dtype=torch.float32)
    beta_out = torch.empty_like(gate_out)
    if batch_size * tokens * value_heads:
        _lib.call(
            "gdn_prepare",
            query.data_ptr(), _lib.i64_array(query.stride()), key.data_ptr(), _lib.i64_array(key.stride()),
            value.data_ptr(), _lib.i64_array(value.stride()), _lib.dtype_code(query.dtype),
            gate.data_ptr(), _lib.i64_array(gate.stride()), _lib.dtype_code(gate.dtype),
            beta.data_ptr(), _lib.i64_array(beta.stride()), _lib.dtype_code(beta.dtype),
            A_log.data_ptr(), A_log.stride(0), _lib.dtype_code(A_log.dtype),
            dt_bias.data_ptr(), dt_bias.stride(0), _lib.dtype_code(dt_bias.dtype),
            batch_size, tokens, key_heads, value_heads, key_dim, value_dim,
            q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), gate_out.data_ptr(), beta_out.data_ptr(),
            _lib.stream_of(query),
        )
    return q_out, k_out, v_out, gate_out, beta_out


__all__ = ["prepare_gdn"]
