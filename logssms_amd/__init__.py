"""MI355X-native (gfx950) Gated DeltaNet hot path for LogSSMs-style hybrid models.

The compute lives in ``libgdn_mi355x.so`` (hand-written HIP, C ABI in
``include/gdn_mi355x.h``); the Python modules below mirror the reference's
operator entry points (same names, argument meaning and error behaviour):

* ``logssms_amd.kernel.prepare_gdn`` / ``store_state``
* ``logssms_amd.kernel.linear_attention.packed_conv.packed_causal_conv1d``
* ``logssms_amd.kernel.linear_attention.conv_decode.conv_decode``
* ``logssms_amd.kernel.linear_attention.gdn`` -- ``chunk_gated_delta_rule_to_cache``,
  ``fused_recurrent_gated_delta_rule_to_slots``, ``fused_recurrent_gated_delta_rule``
* ``logssms_amd.layers.linear_attention_backend.GatedDeltaBackend``
* ``logssms_amd.cache`` -- state pools, Marconi block pool I/O, verify commit.
"""

__all__ = ["kernel", "layers", "cache"]
