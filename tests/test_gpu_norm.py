"""``rms_norm_gated`` (``gdn_rms_norm_gated``, ``csrc/norm.hip``) against the
oracle (``oracle/gdn.py``, pinned in test_oracle.py) on identical inputs.
Outputs are in the io dtype: bf16/f16 rows within rel 2e-2 (plus a small
absolute floor); fp32 rows within 1e-5.  Covers the vector path (widths that
are multiples of 8 up to 512, partly filled lane groups), the one-wave path
(other widths, strided gate columns, fp32 and mixed dtypes), a strided gate
view as the reference's projection split produces, empty input, and HIP
graph replay."""

import pytest
import torch

from oracle import gdn as ref
from tests.gpu_util import DEV, assert_bf16_close, gen, randn

pytestmark = pytest.mark.gpu

CASES = [
    # rows, heads, width, dtype, gate dtype, weight dtype
    (37, 4, 128, torch.bfloat16, torch.bfloat16, torch.float32),
    (16, 2, 64, torch.float16, torch.float16, torch.float32),
    (9, 3, 96, torch.bfloat16, torch.bfloat16, torch.float32),
    (5, 2, 512, torch.bfloat16, torch.bfloat16, torch.float32),
    (7, 2, 8, torch.bfloat16, torch.bfloat16, torch.float32),
    (6, 3, 100, torch.bfloat16, torch.bfloat16, torch.float32),
    (4, 2, 1000, torch.bfloat16, torch.bfloat16, torch.float32),
    (11, 4, 128, torch.float32, torch.float32, torch.float32),
    (8, 4, 128, torch.bfloat16, torch.float16, torch.bfloat16),
]


def _inputs(rows, heads, width, dtype, gdt, wdt, seed, pad=16):
    g = gen(seed)
    x = randn(rows, heads, width, g=g, dtype=dtype)
    # gate as a column slice of a wider projection output, viewed per head
    z = randn(rows, heads * width + pad, g=g, dtype=gdt)[:, :heads * width].view(rows, heads, width)
    w = randn(width, g=g, std=0.5).to(wdt)
    return x, z, w


@pytest.mark.parametrize("case", CASES, ids=[f"r{c[0]}_h{c[1]}_w{c[2]}_{str(c[3])[6:]}" for c in CASES])
def test_rms_norm_gated_matches_oracle(case):
    from logssms_amd.kernel.norm import rms_norm_gated
    rows, heads, width, dtype, gdt, wdt = case
    print(f"rms_norm_gated case {case}", flush=True)
    x, z, w = _inputs(rows, heads, width, dtype, gdt, wdt, 60 + width)
    want = ref.rms_norm_gated(x, z, w, 1e-6)
    got = rms_norm_gated(x.to(DEV), z.to(DEV), w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert got.shape == x.shape and got.dtype == x.dtype
    if dtype == torch.float32:
        torch.testing.assert_close(got.cpu(), want, rtol=1e-5, atol=1e-5)
    else:
        assert_bf16_close(got, want, rel=2e-2, atol=1e-2)


def test_rms_norm_gated_layer_and_strided_gate_columns():
    from logssms_amd.layers import RMSNormGated
    g = gen(71)
    x = randn(10, 4, 128, g=g, dtype=torch.bfloat16)
    zt = randn(4, 128, 10, g=g, dtype=torch.bfloat16)
    z = zt.permute(2, 0, 1)  # column stride != 1: the one-wave path
    norm = RMSNormGated(128, eps=1e-5)
    norm.weight = randn(128, g=g).to(DEV)
    got = norm.forward(x.to(DEV), z.to(DEV))
    assert_bf16_close(got, ref.rms_norm_gated(x, z, norm.weight.cpu(), 1e-5))
    empty = norm.forward(torch.empty(0, 4, 128, device=DEV, dtype=torch.bfloat16),
                         torch.empty(0, 4, 128, device=DEV, dtype=torch.bfloat16))
    assert empty.shape == (0, 4, 128)


def test_rms_norm_gated_graph_replay():
    from logssms_amd.kernel.norm import rms_norm_gated
    x, z, w = _inputs(33, 4, 128, torch.bfloat16, torch.bfloat16, torch.float32, 80)
    x, z, w = x.to(DEV), z.to(DEV), w.to(DEV)
    eager = rms_norm_gated(x, z, w, 1e-6)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        rms_norm_gated(x, z, w, 1e-6)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed = rms_norm_gated(x, z, w, 1e-6)
    for _ in range(3):
        graphed.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graphed, eager)
