"""Linear-attention operators mirroring ``logssms.kernel.linear_attention``
(packed conv, conv decode) and its vendored FLA entry points."""

from .conv_copy import copy_conv_snapshots
from .conv_decode import conv_decode
from .gdn import (
    chunk_gated_delta_rule_to_cache,
    fused_recurrent_gated_delta_rule,
    fused_recurrent_gated_delta_rule_to_logstate,
    fused_recurrent_gated_delta_rule_to_slots,
)
from .logstate import copy_states, restore_log_state_chains, store_log_states
from .packed_conv import PackedConvStateIO, packed_causal_conv1d
from .state_io import ChunkLogIO, ChunkStateIO

__all__ = [
    "ChunkLogIO",
    "ChunkStateIO",
    "PackedConvStateIO",
    "chunk_gated_delta_rule_to_cache",
    "conv_decode",
    "copy_conv_snapshots",
    "copy_states",
    "fused_recurrent_gated_delta_rule",
    "fused_recurrent_gated_delta_rule_to_logstate",
    "fused_recurrent_gated_delta_rule_to_slots",
    "packed_causal_conv1d",
    "restore_log_state_chains",
    "store_log_states",
]
