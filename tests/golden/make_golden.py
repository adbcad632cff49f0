"""Writes ``cfg1_bf16.npz``: BASELINE config 1 (one sequence of 512 tokens,
4 heads, d_k = d_v = 64, chunk 64, zero initial state) with q/k/v rounded to
bf16, solved by the oracle's token recurrence in float64.

Inputs are not stored: ``cfg1_inputs()`` regenerates them from the seed with a
CPU ``torch.Generator``.  Stored: every 8th output row and the final state.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
SEED, T, H, D, EVERY = 1, 512, 4, 64, 8


def cfg1_inputs():
    g = torch.Generator().manual_seed(SEED)
    q = F.normalize(torch.randn(T, H, D, generator=g), dim=-1).to(torch.bfloat16)
    k = F.normalize(torch.randn(T, H, D, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    gate = -torch.rand(T, H, generator=g) * 0.1
    beta = torch.sigmoid(torch.randn(T, H, generator=g))
    return q, k, v, gate, beta


def main():
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    from oracle import gdn as ref
    q, k, v, gate, beta = cfg1_inputs()
    o, s, _ = ref.naive_recurrence(q.double(), k.double(), v.double(), gate.double(), beta.double(), D ** -0.5,
                                   torch.zeros(H, D, D, dtype=torch.float64))
    np.savez(os.path.join(HERE, "cfg1_bf16.npz"), o_rows=o[::EVERY].float().numpy(),
             final_state=s.float().numpy(), meta=np.array([SEED, T, H, D, EVERY]))


if __name__ == "__main__":
    main()
