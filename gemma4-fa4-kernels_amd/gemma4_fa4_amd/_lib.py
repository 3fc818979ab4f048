"""ctypes binding of libgemma4_attn.so (the C ABI declared in include/gemma4_attn.h).

The library is loaded after ``import torch`` so it binds to the HIP runtime
torch already loaded (both carry the soname libamdhip64.so.7); torch's stream
handles and device pointers are then valid for its launches.  A missing library
is an error, never a fallback.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

from .errors import UnsupportedMI355XPath

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libgemma4_attn.so")
ABI_VERSION = 2

G4_OK = 0
G4_ERR_INVALID = 1
G4_ERR_UNSUPPORTED = 2
G4_ERR_WORKSPACE = 3
G4_ERR_LAUNCH = 4
STATIC_WORKSPACE_BYTES = 32 << 20  # G4_STATIC_WORKSPACE_BYTES

EXPORTED_SYMBOLS = (
    "g4_abi_version",
    "g4_last_error",
    "g4_workspace_bytes",
    "g4_attn_fwd",
    "g4_attn_fwd_static",
    "g4_attn_bwd",
    "g4_attn_bwd_delta",
    "g4_attn_bwd_dkdv",
    "g4_attn_bwd_dq",
    "g4_mask_materialize",
    "g4_tile_ranges",
    "g4_kv_prep_fwd",
    "g4_kv_prep_workspace_bytes",
    "g4_kv_prep_bwd",
)


class G4Layout(ctypes.Structure):
    _fields_ = [
        ("batch_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
    ]


class G4Problem(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_k", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("bidirectional_vision", ctypes.c_int32),
        ("total_q", ctypes.c_int64),
        ("total_k", ctypes.c_int64),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("vision_ids", ctypes.c_void_p),
        ("document_ids", ctypes.c_void_p),
        ("lse_batch_stride", ctypes.c_int64),
        ("lse_head_stride", ctypes.c_int64),
        ("ds_budget", ctypes.c_int64),
    ]


class G4KvPrep(ctypes.Structure):
    _fields_ = [
        ("num_batches", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rotary_dim", ctypes.c_int32),
        ("k_fp32", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("cs_batch_stride", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_L = G4Layout
_PROB = ctypes.POINTER(G4Problem)
_PREP = ctypes.POINTER(G4KvPrep)
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "g4_abi_version": (ctypes.c_int, []),
    "g4_last_error": (ctypes.c_char_p, []),
    "g4_workspace_bytes": (ctypes.c_size_t, [_PROB, ctypes.c_int]),
    "g4_attn_fwd": (ctypes.c_int, [_PROB, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _SZ, _P]),
    "g4_attn_fwd_static": (ctypes.c_int, [_PROB, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P]),
    "g4_attn_bwd": (
        ctypes.c_int,
        [_PROB, _P, _L, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _P, _L, _P, _L, _P, _L, _P, _SZ, _P],
    ),
    "g4_attn_bwd_delta": (ctypes.c_int, [_PROB, _P, _L, _P, _L, _P, _P, _SZ, _P]),
    "g4_attn_bwd_dkdv": (
        ctypes.c_int,
        [_PROB, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _L, _P, _L, _P, _SZ, _P],
    ),
    "g4_attn_bwd_dq": (
        ctypes.c_int,
        [_PROB, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _L, _P, _SZ, _P],
    ),
    "g4_mask_materialize": (ctypes.c_int, [_PROB, _P, _P, _SZ, _P]),
    "g4_tile_ranges": (ctypes.c_int, [_PROB, ctypes.c_int, ctypes.c_int, _P, _P, _SZ, _P]),
    "g4_kv_prep_fwd": (ctypes.c_int, [_PREP, _P, _L, _P, _P, _P, _P, _L, _P, _L, _P]),
    "g4_kv_prep_workspace_bytes": (ctypes.c_size_t, [_PREP]),
    "g4_kv_prep_bwd": (
        ctypes.c_int,
        [_PREP, _P, _L, _P, _P, _P, _P, _L, _P, _L, _P, _L, _P, _P, _SZ, _P],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    lib = _lib
    if lib is not None:
        return lib
    with _lock:
        if _lib is not None:
            return _lib
        path = path or LIB_PATH
        if not os.path.exists(path):
            raise UnsupportedMI355XPath(
                f"the gfx950 attention library is not built ({path}); "
                "run __graft_entry__.build() or gemma4-fa4-kernels_amd/build.py"
            )
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.g4_abi_version()
        if version != ABI_VERSION:
            raise UnsupportedMI355XPath(f"library ABI {version} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def device_scope(device: torch.device):
    """A guard that makes ``device`` current for a launch (none when it already is)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def raw_stream(device: torch.device) -> int:
    """The handle of torch's current stream on ``device`` (its ``cuda_stream``)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def check(rc: int) -> None:
    """Raise the Python exception matching a G4_* status code."""
    if rc == G4_OK:
        return
    msg = load().g4_last_error().decode(errors="replace")
    if rc == G4_ERR_INVALID:
        raise ValueError(msg)
    if rc == G4_ERR_UNSUPPORTED:
        raise UnsupportedMI355XPath(msg)
    raise RuntimeError(f"gfx950 attention library error {rc}: {msg}")
