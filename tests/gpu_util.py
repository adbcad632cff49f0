"""Shared helpers for the GPU parity tests (inputs are drawn on the CPU with a
seeded ``torch.Generator`` so the oracle sees the identical values)."""

import torch

DEV = "cuda"


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(*shape, g, dtype=torch.float32, std=1.0):
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def rand(*shape, g, dtype=torch.float32):
    return torch.rand(*shape, generator=g).to(dtype)


def to_dev(*tensors):
    return [t.to(DEV) if isinstance(t, torch.Tensor) else t for t in tensors]


def assert_bf16_close(actual, expected, rel=2e-2, atol=1e-2):
    """bf16 outputs: |a - e| <= atol + rel * |e| elementwise (the north-star
    'rel <= 2e-2' bar, with an absolute floor for values near zero)."""
    a = actual.float().cpu()
    e = expected.float().cpu()
    err = (a - e).abs()
    bound = atol + rel * e.abs()
    bad = err > bound
    assert not bad.any(), (
        f"{int(bad.sum())} / {bad.numel()} elements out of tolerance; max err {float(err.max()):.3e} "
        f"at {tuple(int(i) for i in (bad.nonzero()[0]))}")


def assert_state_close(actual, expected, atol=1e-3):
    """fp32 states: max-abs <= 1e-3."""
    err = (actual.float().cpu() - expected.float().cpu()).abs().max()
    assert float(err) <= atol, f"state max-abs error {float(err):.3e} > {atol}"
