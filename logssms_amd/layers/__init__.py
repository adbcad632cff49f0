"""Layer-level mirrors of ``logssms.layers`` for the GDN path."""

from .gated_delta import GatedDeltaConfig, GatedDeltaNet
from .linear_attention_logstate import (
    GatedDeltaLogStateBackend,
    LogStateLinearAttnCaptureData,
    LogStateLinearAttnMetadata,
)
from .linear_attention_mixed import MixedLinearCopyPlan, prepare_mixed_linear_metadata
from .norm import RMSNormGated

__all__ = ["GatedDeltaConfig", "GatedDeltaLogStateBackend", "GatedDeltaNet", "LogStateLinearAttnCaptureData",
           "LogStateLinearAttnMetadata", "MixedLinearCopyPlan", "RMSNormGated", "prepare_mixed_linear_metadata"]
