"""Fixed-capacity metadata for mixed prefill/decode graph buckets on the CPU
(host paths of ``logssms_amd/layers/linear_attention_mixed.py`` and
``logssms_amd/kernel/metadata.py``): the reference's copy-plan tests
(``tests/layers/test_mixed_metadata_prepare.py:48-75``) and the padding
rules of ``layers/linear_attention_backend/mixed.py:23-120`` as known
answers."""

import pytest
import torch

from logssms_amd.core import Batch, Context, Request
from logssms_amd.kernel.metadata import copy_metadata, pad_metadata
from logssms_amd.layers import GatedDeltaConfig, MixedLinearCopyPlan, prepare_mixed_linear_metadata
from logssms_amd.layers.linear_attention_backend import GatedDeltaBackend


def test_mixed_copy_plan_preserves_strided_guards():
    storage = torch.full((64,), -777)
    destination = {"values": storage[::2], "phase": "decode"}
    plan = MixedLinearCopyPlan(destination)
    source = torch.arange(96)[::3]
    plan.copy({"values": source, "phase": "decode"})
    torch.testing.assert_close(storage[::2], source)
    assert (storage[1::2] == -777).all()


@pytest.mark.parametrize("invalid", ["shape", "constant", "structure"])
def test_mixed_copy_plan_validates_before_writing(invalid):
    first, second = torch.full((4,), -777), torch.full((8,), -777)
    plan = MixedLinearCopyPlan({"tensors": [first, second], "phase": "prefill"})
    source = {"tensors": [torch.ones_like(first), torch.ones_like(second)], "phase": "prefill"}
    if invalid == "shape":
        source["tensors"][1] = torch.ones(7, dtype=second.dtype)
    elif invalid == "constant":
        source["phase"] = "decode"
    else:
        source["tensors"] = tuple(source["tensors"])
    with pytest.raises(ValueError):
        plan.copy(source)
    assert (first == -777).all() and (second == -777).all()


def test_pad_and_copy_metadata_host_rules():
    out = [torch.empty(5, dtype=torch.int64), torch.empty(4, 2, dtype=torch.int64), torch.empty(3, dtype=torch.int32)]
    src = [torch.tensor([1, 2, 3]), torch.tensor([[0, 0], [0, 1]]), torch.tensor([7], dtype=torch.int32)]
    pad_metadata(src, out, [-1, 0, 9], [-1, 128, -1])
    assert out[0].tolist() == [1, 2, 3, -1, -1]
    assert out[1].tolist() == [[0, 0], [0, 1], [0, 128], [0, 128]]
    assert out[2].tolist() == [7, 9, 9]
    dst = [torch.zeros(3, dtype=torch.int64)]
    copy_metadata([torch.tensor([4, 5, 6])], dst)
    assert dst[0].tolist() == [4, 5, 6]
    with pytest.raises(ValueError):
        copy_metadata([torch.tensor([1, 2])], dst)


def _cfg():
    return GatedDeltaConfig(num_k_heads=2, num_v_heads=2, head_k_dim=32, head_v_dim=32, conv_dim=192, state_len=3,
                            layer_idx=0)


def test_prepare_mixed_linear_metadata_pads_to_capacity():
    ctx = Context(page_size=64, state_table=torch.arange(4 * 256, dtype=torch.int32).view(4, 256))
    backend = GatedDeltaBackend(ctx)
    prefill = Batch([Request(0, 0, 70), Request(1, 64, 65)], "prefill")
    decode = Batch([Request(2, 9, 10), Request(3, 0, 1)], "decode")
    backend.prepare_metadata(prefill)
    backend.prepare_metadata(decode)
    actual = prefill.linear_attn_metadata
    before = {name: getattr(actual, name).clone() for name in
              ("chunk_write_slots", "conv_token_slots", "checkpoint_slots", "checkpoint_chunks", "snapshot_rows",
               "snapshot_reqs")}
    cu = actual.prefill_indices.cu_seqlens.clone()
    pm, dm = prepare_mixed_linear_metadata(prefill, decode, 128)
    assert prefill.linear_attn_metadata is pm and decode.linear_attn_metadata is dm
    chunk_capacity = 2 + (128 - 2) // 64  # requests + (capacity - requests) // chunk
    assert pm.chunk_write_slots.shape == (chunk_capacity,) and pm.conv_token_slots.shape == (128,)
    for name, old in before.items():
        new = getattr(pm, name)
        assert torch.equal(new[:len(old)], old), name
        fill = -1 if name in ("chunk_write_slots", "conv_token_slots", "checkpoint_slots") else 0
        assert (new[len(old):] == fill).all(), name
    assert torch.equal(pm.prefill_indices.cu_seqlens, cu)
    chunks = pm.prefill_indices.chunk_indices
    n = len(actual.prefill_indices.chunk_indices)
    assert chunks.shape == (chunk_capacity, 2) and (chunks[n:, 0] == 0).all() and (chunks[n:, 1] == 128).all()
    assert dm.read_slots.dtype == torch.int64 and dm.read_slots.tolist() == [2 * 256 + 8, 3 * 256 + 255]
    backend.prepare_metadata(prefill)
    backend.prepare_metadata(decode)
    with pytest.raises(ValueError, match="exceeds mixed graph capacity"):
        prepare_mixed_linear_metadata(prefill, decode, 64)  # 71 actual tokens


def test_mixed_batch_fields_follow_the_reference():
    reqs = [Request(0, 0, 5), Request(1, 3, 9), Request(2, 7, 8)]
    batch = Batch(reqs, "mixed", num_prefill_reqs=2)
    assert batch.is_mixed and not batch.is_prefill and batch.prefill_count == 2
    assert batch.prefill_reqs == reqs[:2] and batch.decode_reqs == reqs[2:] and batch.prefill_tokens == 11
    assert not Batch(reqs, "prefill").is_mixed and Batch(reqs, "prefill").prefill_count == 3
