"""The stamp tools under logssms_amd/csrc/probe instrument the current kernel
sources: every text they anchor on is still there exactly once, and the
stamped copy carries a stamp on each side of every loop barrier.  CPU only
(a text transform; building and running the copies needs hipcc and a GPU)."""

import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = os.path.join(ROOT, "logssms_amd", "csrc", "probe")
CSRC = os.path.join(ROOT, "logssms_amd", "csrc")


def _load(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(PROBE, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_chunk_stamps_instrument_current_source():
    tool = _load("chunk_stamps")
    src = open(os.path.join(CSRC, "chunk_chain.hip")).read()
    out = tool.instrument(src)
    # 4 roles x (1 before M, 1 after M, 1 before B, 1 after B) + the fused conv waves' peeled chunk
    for k in (1, 2, 3, 4):
        assert out.count("STAMP(%d);" % k) == 5, k
    assert out.count("const int64_t c = nchunks - 1;") == 1
    assert "gdn_stamps_read" in out and "stamps_hwid_kernel" in out
    # the product source itself is untouched
    assert "STAMP(" not in src


def test_logstate_stamps_instrument_current_source():
    tool = _load("logstate_stamps")
    src = open(os.path.join(CSRC, "logstate.hip")).read()
    out = tool.instrument(src)
    assert out.count("LSTAMP(0);") == 2  # loading and compute head loops
    assert out.count("LSTAMP(1);") == 1 and out.count("LSTAMP(2);") == 1
    for k in (3, 4, 5, 6):
        assert out.count("LSTAMP(%d);" % k) == 2, k
    assert "gdn_lsstamps_read" in out
    assert "LSTAMP(" not in src


def test_stamp_tools_reject_a_changed_source():
    tool = _load("chunk_stamps")
    src = open(os.path.join(CSRC, "chunk_chain.hip")).read()
    with pytest.raises(SystemExit):
        tool.instrument(src.replace("lds_barrier();  // M(c)", "lds_barrier();  // M", 1))
