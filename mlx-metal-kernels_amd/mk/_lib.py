"""ctypes binding of libmk_hip.so (the gfx950 kernels) for torch tensors.

The shared library exports a plain C ABI (``include/mk_hip.h``).  This module
loads it once, declares every entry point's signature, and offers ``launch``,
which passes raw device pointers plus the current HIP stream of the tensors'
device and turns a negative status into ``RuntimeError``.

``torch`` must be imported before the library is loaded: torch ships its own
``libamdhip64.so.7`` and the library has to bind to that same HIP runtime
instance (same SONAME), so that pointers and streams created by torch are
valid inside the kernels.

There is no fallback: if the library is missing or the tensors are not on a
ROCm device, every non-``reference`` backend raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libmk_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

MK_OK = 0
MK_ERR_INVALID = -1
MK_ERR_UNSUPPORTED = -2
MK_ERR_SCRATCH = -3

DT_F16 = 0
DT_BF16 = 1
DT_F32 = 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double
_SZ = ctypes.c_size_t

# name -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "mk_abi_version": [],
    "mk_pack_q4": [_P, _P, _I64, _I64, _P],
    "mk_unpack_q4": [_P, _P, _I64, _I64, _I64, _P],
    "mk_dequant_q4": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P],
    "mk_dequant_q8": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P],
    "mk_quantize_weight": [_P, _P, _P, _I64, _I64, _I64, _I, _D, _I, _I, _P],
    "mk_q4_matvec": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P],
    "mk_q8_matvec": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P],
    "mk_q4_gate_up": [_P] * 10 + [_I64] * 4 + [_I, _I, _P],
    "mk_q8_gate_up": [_P] * 10 + [_I64] * 4 + [_I, _I, _P],
    "mk_argmax_rows": [_P, _P, _I64, _I64, _I, _P],
    "mk_q4_rmsnorm_qkv_rope_paged": [_P, _P, _F] + [_P] * 12 + [_I64] * 10 + [_I, _I, _I, _P],
    "mk_q8_rmsnorm_qkv_rope_paged": [_P, _P, _F] + [_P] * 12 + [_I64] * 10 + [_I, _I, _I, _P],
    "mk_q4_rmsnorm_matvec": [_P, _P, _F] + [_P] * 5 + [_I64] * 4 + [_I, _I, _I, _P],
    "mk_q8_rmsnorm_matvec": [_P, _P, _F] + [_P] * 5 + [_I64] * 4 + [_I, _I, _I, _P],
    "mk_q4_rmsnorm_gate_up": [_P, _P, _P, _F] + [_P] * 11 + [_I64] * 4 + [_I, _I, _I, _P],
    "mk_q8_rmsnorm_gate_up": [_P, _P, _P, _F] + [_P] * 11 + [_I64] * 4 + [_I, _I, _I, _P],
    "mk_swiglu": [_P, _P, _P, _I64, _I, _P],
    "mk_residual_add": [_P, _P, _P, _I64, _I, _P],
    "mk_rms_norm": [_P, _P, _P, _I64, _I64, _F, _I, _I, _P],
    "mk_residual_rms_norm": [_P, _P, _P, _P, _P, _I64, _I64, _F, _I, _I, _P],
    "mk_block_table_lookup": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "mk_paged_kv_update": [_P, _P, _P, _P, _P, _P] + [_I64] * 6 + [_I, _P],
    "mk_qkv_rope_paged_update": [_P] * 8 + [_I64] * 8 + [_I, _P],
    "mk_qkv_rope_paged_update_quant": [_P] * 10 + [_I64] * 9 + [_I, _I, _P],
    "mk_quantize_kv": [_P, _P, _P, _I64, _I64, _I64, _I, _I, _P],
    "mk_paged_attention_workspace_bytes": [_I64] * 6,
    "mk_paged_decode_attention": [_P] * 6 + [_I64] * 7 + [_F, _I, _P, _SZ, _P],
    "mk_paged_decode_attention_noalloc": [_P] * 6 + [_I64] * 7 + [_F, _I, _P],
    "mk_paged_quantized_decode_attention": [_P] * 8 + [_I64] * 8 + [_I, _F, _I, _P, _SZ, _P],
    "mk_paged_verify_attention": [_P] * 6 + [_I64] * 8 + [_F, _I, _P, _SZ, _P],
    "mk_paged_quantized_verify_attention": [_P] * 8 + [_I64] * 9 + [_I, _F, _I, _P, _SZ, _P],
}
_RESTYPES = {"mk_paged_attention_workspace_bytes": _SZ}

_lock = threading.Lock()
_lib = None


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or cannot be loaded."""


# mk_abi_version() of the library these signatures describe
ABI_VERSION = 2


def library_path() -> Path:
    override = os.environ.get("MK_HIP_LIBRARY")
    return Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises NativeLibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise NativeLibraryError(
                f"{path} is not built; run `make -C mlx-metal-kernels_amd` "
                "(or __graft_entry__.build()) before using a HIP backend"
            )
        lib = ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, _I)
        found = lib.mk_abi_version()
        if found != ABI_VERSION:
            raise NativeLibraryError(
                f"{path} has ABI version {found}, this binding expects {ABI_VERSION}; rebuild the library"
            )
        _lib = lib
        return lib


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return DT_F16
    if dtype == torch.bfloat16:
        return DT_BF16
    if dtype == torch.float32:
        return DT_F32
    raise TypeError(f"unsupported dtype {dtype}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def require_device(*tensors) -> torch.device:
    """All given tensors must sit on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError(
                f"HIP backends need tensors on a ROCm device, got a tensor on {t.device}; "
                "use backend='reference' for host tensors"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors are on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def launch(name: str, device: torch.device, *args) -> int:
    """Call ``name`` with ``args`` on the current stream of ``device``."""
    lib = load()
    fn = getattr(lib, name)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = fn(*args, ctypes.c_void_p(stream))
    if rc != MK_OK:
        if rc == MK_ERR_INVALID:
            raise RuntimeError(f"{name}: invalid argument (status {rc})")
        if rc == MK_ERR_UNSUPPORTED:
            raise RuntimeError(f"{name}: unsupported shape/dtype combination (status {rc})")
        if rc == MK_ERR_SCRATCH:
            raise RuntimeError(f"{name}: the call needs more than the library's fixed 16 MiB "
                               f"no-allocation scratch (status {rc}); use the workspace entry point")
        raise RuntimeError(f"{name}: HIP launch failed (hipError {-rc - 1000})")
    return rc


def workspace_bytes(B: int, Hq: int, Hkv: int, D: int, max_blocks: int, page_size: int) -> int:
    return int(load().mk_paged_attention_workspace_bytes(B, Hq, Hkv, D, max_blocks, page_size))


# Zero-filled workspaces, one per (kind, device, stream).  The library keeps
# the attention's arrival counters at the start of a workspace: they must be
# zero before a call and every call leaves them zero, so one buffer serves
# every call issued on its stream (calls on one stream never overlap).
# A graph captured on a stream keeps using the buffer handed out during the
# capture: such a buffer, once replaced by a larger one, is retired (kept
# alive) rather than freed; any other replaced buffer is freed.  Graphs that
# captured on the same stream share its buffer, so they must be replayed on
# one stream, one after another (the decode graphs and bench.py do this).
_WORKSPACES: dict = {}
_RETIRED: list = []
_CAPTURED: set = set()
_WS_LOCK = threading.Lock()


def _stream_workspace(kind: str, device: torch.device, nbytes: int):
    size = (nbytes + 255) // 256 * 256
    dev = torch.device(device)
    key = (kind, dev.index, torch.cuda.current_stream(dev).cuda_stream)
    capturing = torch.cuda.is_current_stream_capturing()
    with _WS_LOCK:
        buf = _WORKSPACES.get(key)
        if buf is None or buf.numel() < size:
            old = buf
            buf = torch.zeros(size, dtype=torch.uint8, device=dev)
            if capturing:  # made inside the capture: the graph zero-fills it on every replay
                return buf
            if old is not None and old.data_ptr() in _CAPTURED:
                _RETIRED.append(old)
            _WORKSPACES[key] = buf
        if capturing:
            _CAPTURED.add(buf.data_ptr())
    return buf


def attention_workspace(device: torch.device, B: int, Hq: int, Hkv: int, D: int, max_blocks: int,
                        page_size: int):
    """(workspace, nbytes) for one paged-attention call on the current stream
    of ``device``: the stream's zero-filled workspace, replaced by a larger
    one when the call needs more.  Under graph capture with no large enough
    buffer cached, a new zero-filled buffer is made for the captured call
    (the graph then zero-fills it on every replay)."""
    nbytes = workspace_bytes(B, Hq, Hkv, D, max_blocks, page_size)
    if nbytes <= 0:
        return None, 0
    return _stream_workspace("attention", device, nbytes), nbytes

