"""CPU checks of the C ABI: the built library loads, exports every entry point
declared in include/gdn_mi355x.h, and the ctypes table matches the header's
parameter types one by one (no compute call is made)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gdn_mi355x.h")


def _declarations():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for m in re.finditer(r"(?:int64_t|int|const char\*)\s+(gdn_\w+)\s*\(([^;]*?)\);", src, re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = params
    return out


def _ctype_of(param):
    decl = re.sub(r"\s+", " ", param)
    if "int64_t*" in decl.replace(" ", ""):
        return ctypes.POINTER(ctypes.c_int64)
    if "*" in decl:
        return ctypes.c_void_p
    if decl.startswith("int64_t"):
        return ctypes.c_int64
    if decl.startswith("int "):
        return ctypes.c_int
    if decl.startswith("float"):
        return ctypes.c_float
    raise AssertionError(f"unmapped parameter type: {param}")


def test_header_declares_expected_entry_points():
    names = set(_declarations())
    assert {"gdn_last_error", "gdn_abi_version", "gdn_chunk_gated_delta_rule", "gdn_fused_recurrent",
            "gdn_fused_conv_recurrent", "gdn_packed_causal_conv1d", "gdn_prepare", "gdn_prefill_frontend",
            "gdn_conv_decode", "gdn_store_state", "gdn_copy_rows", "gdn_zero_rows",
            "gdn_commit_accepted", "gdn_prefill_qk", "gdn_prefill_fused", "gdn_conv_snapshots",
            "gdn_rms_norm_gated", "gdn_metadata_copy", "gdn_metadata_pad", "gdn_prefill_fused_noalloc",
            "gdn_prefill_noalloc_scratch_bytes", "gdn_gather_linear_slots"} <= names
    assert "gdn_probe_rmw" not in names  # the bench-only probe lives in libgdn_probe.so


def test_ctypes_table_matches_header():
    from logssms_amd import _lib
    decls = _declarations()
    for name, params in decls.items():
        if name in ("gdn_last_error", "gdn_abi_version", "gdn_prefill_noalloc_scratch_bytes"):
            assert params == []
            continue
        assert name in _lib.SIGNATURES, name
        want = [_ctype_of(p) for p in params]
        assert _lib.SIGNATURES[name] == want, name


def test_library_loads_and_exports_every_symbol():
    from logssms_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.lib()
    for name in _declarations():
        assert hasattr(lib, name), name
    assert lib.gdn_abi_version() == 6
    assert lib.gdn_prefill_noalloc_scratch_bytes() == 256 << 20
    assert lib.gdn_last_error() in (b"",) or isinstance(lib.gdn_last_error(), bytes)


def test_invalid_arguments_report_errors_without_a_gpu():
    """Argument validation happens before any HIP call, so it runs on a CPU box."""
    from logssms_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.lib()
    rc = lib.gdn_store_state(None, 0, None, 5, None, 0, 3, 128, None)
    assert rc == 1
    assert b"indices" in lib.gdn_last_error()
    rc = lib.gdn_fused_conv_recurrent(*([None, 0, 0, 1, None, 0, None, None, 4, None, 0, 0, 1, None, 0, 0, 1, None,
                                         0, None, 0, 1, 17, 2, 4, 64, 64, None, 0, 0, None, 0, 0, 0, 0, 0, None, 0,
                                         1, None, 0, 1, 1, None, 1.0, None]))
    assert rc == 1
    assert b"steps" in lib.gdn_last_error()
    # empty work is a no-op success
    assert lib.gdn_copy_rows(None, 0, None, 1, None, 0, None, 1, 0, 1, 16, 0, None) == 0
    assert lib.gdn_rms_norm_gated(None, 1, 0, 128, None, 1, 32, 4096, 128, 1, None, 0, 1e-6, None, None) == 0
    assert lib.gdn_rms_norm_gated(None, 1, 4, 0, None, 1, 32, 4096, 128, 1, None, 0, 1e-6, None, None) == 1
    assert b"bad shape" in lib.gdn_last_error()
    assert lib.gdn_rms_norm_gated(None, 7, 4, 128, None, 1, 32, 4096, 128, 1, None, 0, 1e-6, None, None) == 1
    assert lib.gdn_rms_norm_gated(None, 1, 4, 128, None, 1, 32, 4096, 128, 1, None, 0, 1e-6, None, None) == 1
    assert b"null" in lib.gdn_last_error()
    assert lib.gdn_metadata_copy(None, None, None, None, None, None, 0, None) == 0  # nothing to move
    assert lib.gdn_metadata_pad(None, None, None, None, None, None, None, 0, None) == 0
    assert lib.gdn_metadata_pad(None, None, None, None, None, None, None, 2, None) == 1
    assert b"null table" in lib.gdn_last_error()


def test_fused_prefill_reports_uncovered_shapes_without_launching():
    """gdn_prefill_qk / gdn_prefill_fused check their coverage on the host and
    return GDN_ERR_UNSUPPORTED (the caller then takes the two-step path)
    before any HIP call; the dummy device pointers are never dereferenced."""
    from logssms_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.lib()
    d = 0x10000  # 16-byte aligned dummy address

    def qk(width, dk, row_stride=8192):
        return lib.gdn_prefill_qk(d, row_stride, 1, d, width, d, 1, 1, 64, 16, dk, d, 0, 0, 0, d, 1, d, d, 2, 32,
                                  d, 32, 1, 1, d, 32, 1, 1, d, 0, d, 0, d, d, None)

    def fused(width, dk, dv, row_stride=8192):
        return lib.gdn_prefill_fused(d, d, d, row_stride, 1, d, width, d, 1, 1, 64, 16, 32, dk, dv, d, 0, 0, d, d, d,
                                     0, 0, 0, 0, 0, d, 1, d, 1, None, 1, None, 0, None, 0, 0, d, 0.1, None)
    assert qk(3, 128) == 2
    assert b"not covered" in lib.gdn_last_error()
    assert qk(4, 256) == 2
    assert qk(4, 128, row_stride=8190) == 2
    assert fused(3, 128, 128) == 2
    assert b"not covered" in lib.gdn_last_error()
    assert fused(4, 128, 96) == 2
    assert lib.gdn_conv_snapshots(d, 8192, 0, d, 1, 1, 64, 8192, 4, d, 0, 0, 0, d, 1, d, 1, d, 1, 4, None) == 1
