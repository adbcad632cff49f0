"""``GatedDeltaConfig`` and the ``GatedDeltaNet`` layer (reference
``python/logssms/layers/gated_delta.py:15-139``) on one GPU.

The layer is the boundary either side of the GDN path: the merged input
projections whose column slices feed the conv and the gates as strided views
(no copies), the backend call, and the gated RMS norm plus output projection.
With one GPU the column- and row-parallel linears are plain GEMMs
(``torch.nn.functional.linear``, i.e. hipBLASLt); the tensor-parallel head
split and the row-parallel all-reduce are not part of this build."""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .norm import RMSNormGated


@dataclass(frozen=True)
class GatedDeltaConfig:
    num_k_heads: int
    num_v_heads: int
    head_k_dim: int
    head_v_dim: int
    conv_dim: int
    state_len: int
    layer_idx: int

    @property
    def key_dim(self) -> int:
        return self.num_k_heads * self.head_k_dim

    @property
    def value_dim(self) -> int:
        return self.num_v_heads * self.head_v_dim


class GatedDeltaNet:
    """``GatedDeltaNet`` (``layers/gated_delta.py:44-139``).  Parameters carry
    the reference's shapes: ``in_proj_qkvz_weight [conv_dim + value_dim,
    hidden]``, ``in_proj_ba_weight [2 HV, hidden]``, ``conv1d_weight
    [conv_dim, 1, W]``, ``dt_bias [HV]`` (ones), ``A_log [HV]`` (fp32 zeros),
    ``norm.weight [head_v_dim]`` (fp32 ones), ``out_proj_weight [hidden,
    value_dim]``; the projections are left uninitialised, as there."""

    def __init__(
        self,
        hidden_size: int,
        num_key_heads: int,
        num_value_heads: int,
        head_k_dim: int,
        head_v_dim: int,
        conv_kernel_size: int,
        rms_norm_eps: float,
        layer_idx: int,
        *,
        device=None,
        dtype: torch.dtype | None = None,
    ):
        key_dim = num_key_heads * head_k_dim
        value_dim = num_value_heads * head_v_dim
        conv_dim = key_dim * 2 + value_dim
        self._config = GatedDeltaConfig(
            num_k_heads=num_key_heads, num_v_heads=num_value_heads, head_k_dim=head_k_dim,
            head_v_dim=head_v_dim, conv_dim=conv_dim, state_len=conv_kernel_size - 1, layer_idx=layer_idx,
        )
        self._linear_layer_idx = layer_idx
        kw = dict(device=device, dtype=dtype)
        self.conv1d_weight = torch.empty(conv_dim, 1, conv_kernel_size, **kw)
        self.dt_bias = torch.ones(num_value_heads, **kw)
        self.A_log = torch.zeros(num_value_heads, dtype=torch.float32, device=device)
        self.norm = RMSNormGated(head_v_dim, eps=rms_norm_eps)
        self.norm.weight = self.norm.weight.to(device)
        self.out_proj_weight = torch.empty(hidden_size, value_dim, **kw)
        self.in_proj_qkvz_weight = torch.empty(conv_dim + value_dim, hidden_size, **kw)
        self.in_proj_ba_weight = torch.empty(2 * num_value_heads, hidden_size, **kw)

    @property
    def config(self) -> GatedDeltaConfig:
        return self._config

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        mixed_qkv, z, beta, gate = self.proj(x)
        core_output = self.attend(mixed_qkv, beta, gate)
        return self.output(core_output, z)

    def proj(self, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """``:99-105``: column slices of the two projections, as views."""
        config = self._config
        mixed_qkv, z = F.linear(x, self.in_proj_qkvz_weight).split([config.conv_dim, config.value_dim], dim=-1)
        beta, gate = F.linear(x, self.in_proj_ba_weight).chunk(2, dim=-1)
        return mixed_qkv, z, beta, gate

    def attend(self, mixed_qkv: torch.Tensor, beta: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        """``:107-131``: the backend of the global context on the context's batch
        (a mixed batch through ``forward_mixed``)."""
        from ..core import get_global_ctx

        ctx = get_global_ctx()
        if ctx.batch.is_mixed:
            return ctx.linear_attn_backend.forward_mixed(
                ctx.batch, {"mixed_qkv": mixed_qkv, "gate": gate, "beta": beta},
                conv_weight=self.conv1d_weight, A_log=self.A_log, dt_bias=self.dt_bias, config=self._config,
            )
        return ctx.linear_attn_backend.forward(
            mixed_qkv=mixed_qkv, gate=gate, beta=beta, conv_weight=self.conv1d_weight, A_log=self.A_log,
            dt_bias=self.dt_bias, config=self._config, batch=ctx.batch,
        )

    def output(self, core_output: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
        """``:133-139``: gated RMS norm per v-head, then the output projection."""
        config = self._config
        shape = (core_output.shape[0], config.num_v_heads, config.head_v_dim)
        output = self.norm.forward(core_output.reshape(shape), z.view(shape)).reshape(core_output.shape[0], -1)
        return F.linear(output, self.out_proj_weight)


__all__ = ["GatedDeltaConfig", "GatedDeltaNet"]
