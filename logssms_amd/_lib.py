"""Loader for ``libgdn_mi355x.so`` (the gfx950 HIP kernels behind the C ABI
declared in ``include/gdn_mi355x.h``).

There is no fallback: if the library is missing or a call fails, a
``RuntimeError`` is raised.  Tensors are passed as raw device pointers; the
launch goes on torch's current stream of the tensor's device.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgdn_mi355x.so")

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
PI64 = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (restype is always int)
SIGNATURES = {
    "gdn_packed_causal_conv1d": [P, I64, I64, I32, P, P, P, P, I32, I64, I64, I64, I32, P, P, I64, I64, I64,
                                 P, I32, P, I32, I64, I64, F32, F32, F32, P],
    "gdn_prepare": [P, PI64, P, PI64, P, PI64, I32, P, PI64, I32, P, PI64, I32, P, I64, I32, P, I64, I32,
                    I64, I64, I64, I64, I64, I64, P, P, P, P, P, P],
    "gdn_prefill_frontend": [P, I64, I64, I32, P, P, I32, P, I32, I64, I64, I64, I64, I64, I64, P, I64, I64,
                             I64, P, I32, P, I64, I64, I32, P, I64, I64, I32, P, I32, P, I32, P, P,
                             P, P, P, P],
    "gdn_prefill_qk": [P, I64, I32, P, I32, P, I32, I64, I64, I64, I64, P, I64, I64, I64, P, I32, P, P, I32, I64,
                       P, I64, I64, I32, P, I64, I64, I32, P, I32, P, I32, P, P, P],
    "gdn_prefill_fused": [P, P, P, I64, I32, P, I32, P, I32, I64, I64, I64, I64, I64, I64, P, I64, I64, P, P, P, I32,
                          I64, I64, I64, I64, P, I32, P, I32, P, I32, P, I32, P, I32, I64, P, F32, P],
    "gdn_metadata_copy": [P, P, PI64, PI64, PI64, P, I32, P],
    "gdn_metadata_pad": [P, P, PI64, PI64, PI64, PI64, P, I32, P],
    "gdn_rms_norm_gated": [P, I32, I64, I64, P, I32, I64, I64, I64, I64, P, I32, F32, P, P],
    "gdn_conv_snapshots": [P, I64, I32, P, I32, I64, I64, I64, I32, P, I64, I64, I64, P, I32, P, I32, P, I32, I64,
                           P],
    "gdn_chunk_gated_delta_rule": [P, P, P, I32, P, P, P, I32, I64, I64, I64, I64, I64, I64, P, I32, I64, I64, I64,
                                   I64, P, I32, P, I32, P, I32, I64, P, I32, I64, I64, I64, I64, I64, P, P, F32, P],
    "gdn_chunk_gated_delta_rule_logged": [P, P, P, I32, P, P, P, I32, I64, I64, I64, I64, I64, I64, P, I32, I64, P,
                                          I32, P, I32, P, I32, I64, P, I32, I64, I64, I64, I64, I64, P, I32, P, I32,
                                          I64, I64, I64, P, F32, P],
    "gdn_store_chunk_log": [P, P, I32, I64, I64, I64, I64, P, I32, P, I32, I64, P, P, I64, I64, I64, I64, I64, P, P,
                            I32, I64, I64, I64, I64, I64, P],
    "gdn_conv_windows_logstate": [P, I64, I64, I32, P, P, I32, I64, I64, I64, I32, P, P, I32, I64, I64, I64, I64,
                                  I64, I64, P, I32, P, I32, P, I32, I64, I64, F32, F32, F32, P],
    "gdn_logstate_copy_conv": [P, P, I32, I64, I64, I64, I64, I64, I64, P, I32, P, I32, P, I32, P, I32, I64, P],
    "gdn_logstate_store_conv": [P, P, I32, I64, I64, I64, I64, I64, P, I32, P, I32, I64, I64, I64, P, P],
    "gdn_logstate_store_states": [P, P, I32, I64, I64, I64, I64, I64, P, I32, I64, I64, I64, I64, P, P],
    "gdn_logstate_prefill_writes": [P, I32, P, I32, P, P, I64, I64, P],
    "gdn_gather_linear_slots": [P, I32, P, I32, P, I32, I64, I64, I64, P, I32, I64, I64, P, I32, I64, P, I64, P],
    "gdn_logstate_restore": [P, P, I32, I64, I64, I64, I64, I64, P, I32, I64, I64, I64, I64, I64, I64, I64, I64,
                             I32, P, P, P, P, P, P, I64, P],
    "gdn_logstate_copy_states": [P, P, I32, I64, I64, I64, I64, I64, I64, I64, I64, I64, I32, P, P, I64, P],
    "gdn_conv_decode_logstate": [P, I64, I64, I32, P, P, I32, I64, I64, P, P, I32, I64, I64, I64, I64, I64, I64, P,
                                 I32, P, I32, P, I32, P, I32, P, I32, P, P, P, I64, I32, I32, I64, I64, F32, F32,
                                 F32, P],
    "gdn_recurrent_logstate": [P, P, P, I32, P, I64, I64, I32, P, I64, I64, I32, P, I32, P, I32, I64, I64, I64, I64,
                               I64, P, P, I32, I64, I64, I64, I64, I64, P, I32, I64, P, I32, P, I32, P, I32, P, I32,
                               I64, I64, I64, I64, I32, P, F32, P],
    "gdn_conv_decode": [P, I64, I64, I32, P, P, I32, I64, I64, P, I64, I64, I64, P, I64, I32, P, I64, I32, P,
                        P, P, I64, I32, I32, I64, I64, F32, F32, F32, P],
    "gdn_fused_recurrent": [P, P, P, I32, P, I64, I64, I64, I32, P, I64, I64, I64, I32, P, I32, P, I32, I64,
                            I64, I64, I64, I64, I64, P, I32, I64, I64, I64, I64, P, I64, I32, P, I64, I64,
                            I32, P, P, P, F32, P],
    "gdn_fused_conv_recurrent": [P, I64, I64, I32, P, I32, P, P, I32, P, I64, I64, I32, P, I64, I64, I32, P,
                                 I32, P, I32, I64, I64, I64, I64, I64, I64, P, I64, I64, P, I32, I64, I64, I64,
                                 I64, P, I64, I32, P, I64, I64, I32, P, F32, P],
    "gdn_store_state": [P, I64, P, I32, P, I64, I64, I64, P],
    "gdn_copy_rows": [P, I64, P, I32, P, I64, P, I32, I64, I64, I64, I64, P],
    "gdn_zero_rows": [P, I64, P, I32, I64, I64, I64, I64, P],
    "gdn_prefill_fused_noalloc": [P, I64, I32, P, I32, P, I32, I64, I64, I64, I64, I64, I64, P, I64, I64, P, I64,
                                  I64, I32, P, I64, I64, I32, P, I32, P, I32, P, I32, I64, I64, I64, I64, P, I32,
                                  P, I32, P, I32, P, I32, I64, P, F32, P],
    "gdn_commit_accepted": [P, I64, I64, I64, P, I64, I64, I64, P, I32, P, I64, I64, I32, P, I32, I64, I64, P],
}

F32_CODE, BF16_CODE, F16_CODE = 0, 1, 2
I32_CODE, I64_CODE = 0, 1

_DTYPE_CODES = {torch.float32: F32_CODE, torch.bfloat16: BF16_CODE, torch.float16: F16_CODE}

_lib = None


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C logssms_amd/csrc`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        handle.gdn_last_error.argtypes = []
        handle.gdn_last_error.restype = ctypes.c_char_p
        handle.gdn_abi_version.argtypes = []
        handle.gdn_abi_version.restype = ctypes.c_int
        handle.gdn_prefill_noalloc_scratch_bytes.argtypes = []
        handle.gdn_prefill_noalloc_scratch_bytes.restype = ctypes.c_int64
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise ``RuntimeError`` with the library's message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().gdn_last_error().decode(errors="replace")
        if rc == 2:
            raise NotImplementedError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def index_code(t: torch.Tensor) -> int:
    if t.dtype == torch.int64:
        return I64_CODE
    if t.dtype == torch.int32:
        return I32_CODE
    raise TypeError(f"index tensors must be int32 or int64, got {t.dtype}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    if not t.is_cuda:
        raise RuntimeError("libgdn_mi355x kernels need tensors on a ROCm device")
    return torch.cuda.current_stream(t.device).cuda_stream


def i64_array(values):
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr
