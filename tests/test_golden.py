"""The committed config-1 fixture (``tests/golden/cfg1_bf16.npz``) against the
oracle: the chunked restatement in float64 and the token recurrence in fp32
must both reproduce it."""

import os

import numpy as np
import torch

from oracle import gdn as ref
from tests.golden.make_golden import D, EVERY, H, SEED, T, cfg1_inputs

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "cfg1_bf16.npz")


def load_fixture():
    z = np.load(FIXTURE)
    assert z["meta"].tolist() == [SEED, T, H, D, EVERY]
    return torch.from_numpy(z["o_rows"]), torch.from_numpy(z["final_state"])


def test_chunked_oracle_reproduces_fixture():
    o_rows, state = load_fixture()
    q, k, v, gate, beta = cfg1_inputs()
    o, _, _, s = ref.chunk_gdn(q.double(), k.double(), v.double(), gate.double(), beta.double(), D ** -0.5,
                               torch.zeros(H, D, D, dtype=torch.float64), rcp_ln2=1 / np.log(2))
    torch.testing.assert_close(o[::EVERY].float(), o_rows, rtol=0, atol=1e-6)
    torch.testing.assert_close(s.float(), state, rtol=0, atol=1e-6)


def test_fp32_recurrence_within_state_bar():
    o_rows, state = load_fixture()
    q, k, v, gate, beta = cfg1_inputs()
    o, s, _ = ref.naive_recurrence(q.float(), k.float(), v.float(), gate, beta, D ** -0.5, torch.zeros(H, D, D))
    assert float((s - state).abs().max()) < 1e-4
    assert float((o[::EVERY] - o_rows).abs().max()) < 1e-4
