"""ctypes binding of libpbgdn.so (the C ABI declared in include/pbgdn.h).

torch is imported first so that its HIP runtime is the one in the process:
the library links libamdhip64 by soname and binds to whatever is loaded.
A missing or stale library raises; there is no fallback.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpbgdn.so")
# The debug build of the same sources (build.py): LDS and outputs poisoned with NaN.
DEBUG_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpbgdn_debug.so")
ABI_VERSION = 14

F32, BF16, F16 = 0, 1, 2
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_LAUNCH, ERR_SCRATCH = 0, 1, 2, 3, 4
STATE_STREAM, STATE_RESIDENT = 0, 1  # PBGDN_STATE_*: a decode step's state cache policy
NOALLOC_SCRATCH_BYTES = 64 << 20  # PBGDN_NOALLOC_SCRATCH_BYTES

DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

# Every function the header declares, with its ctypes signature.
_vp, _i, _f, _l = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_long
SIGNATURES = {
    "pbgdn_abi_version": ([], _i),
    "pbgdn_status_string": ([_i], ctypes.c_char_p),
    "pbgdn_chunk_fwd": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i,
                         _i, _i, _i, _i, _i, _i, _f, _i, _vp, ctypes.c_size_t, _vp], _i),
    "pbgdn_chunk_layer_fwd": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _i,
                               _vp, _l, _i, _vp, _f, _vp, _i, _vp,
                               _i, _i, _i, _i, _i, _i, _f, _i, _vp, ctypes.c_size_t, _vp], _i),
    "pbgdn_chunk_workspace_size": ([_i, _i, _i, _i, _i], ctypes.c_size_t),
    "pbgdn_chunk_layer_fuses": ([_i, _i, _i, _l, _i, _i, _i, _i], _i),
    "pbgdn_chunk_fwd_noalloc": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i,
                                 _i, _i, _i, _i, _i, _i, _f, _i, _vp], _i),
    "pbgdn_recurrent_fwd": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i,
                             _i, _i, _i, _i, _i, _i, _f, _i, _vp], _i),
    "pbgdn_recurrent_verify_fwd": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _i,
                                    _i, _i, _i, _i, _i, _i, _f, _vp], _i),
    "pbgdn_prologue_fwd": ([_vp, _l, _vp, _l, _i, _vp, _vp, _i, _vp, _i, _vp, _vp,
                            _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp], _i),
    "pbgdn_epilogue_fwd": ([_vp, _i, _vp, _l, _i, _vp, _f, _vp, _i, _i, _i, _i, _i, _vp], _i),
    "pbgdn_prologue_varlen_fwd": ([_vp, _l, _vp, _l, _i, _vp, _i, _vp, _vp, _i, _l, _l, _l, _vp, _vp, _i,
                                   _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp],
                                  _i),
    "pbgdn_decode_layer_fwd": ([_vp, _l, _i, _vp, _i, _l, _l, _l, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i,
                                _vp, _f, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp], _i),
    "pbgdn_chunk_bwd": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                         _vp, ctypes.c_size_t, _i, _i, _i, _i, _i, _i, _f, _vp], _i),
    "pbgdn_chunk_bwd_workspace_size": ([_i, _i, _i, _i, _i, _i], ctypes.c_size_t),
    "pbgdn_chunk_residuals": ([_vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp], _i),
    "pbgdn_chunk_decumulate": ([_vp, _vp, _i, _i, _i, _vp], _i),
    "pbgdn_stream_probe": ([_vp, _vp, ctypes.c_int64, _vp], _i),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class PbgdnError(RuntimeError):
    """A nonzero status returned by the C ABI."""

    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: pbgdn status {status}: {status_string(status)}")


def _load(path: str) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(
            f"pbgdn HIP library not found at {path}; build it with "
            "`python -m pseudobrain_amd.build` (there is no CPU fallback)")
    handle = ctypes.CDLL(path)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = res
    version = handle.pbgdn_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{os.path.basename(path)} ABI version {version}, expected {ABI_VERSION}; rebuild it")
    return handle


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            _lib = _load(LIB_PATH)
    return _lib


_debug: ctypes.CDLL | None = None


@contextlib.contextmanager
def debug_library():
    """Within the block every call of this package goes to libpbgdn_debug.so,
    whose kernels fill their LDS with NaN before use and whose entry points
    fill their outputs and workspaces with NaN before launching (a test aid:
    an unwritten output element or a read of unwritten LDS then shows as NaN).
    Not thread-safe: the other library is restored on exit."""
    global _lib, _debug
    prev = lib()
    if _debug is None:
        _debug = _load(DEBUG_LIB_PATH)
    _lib = _debug
    try:
        yield _debug
    finally:
        _lib = prev


def status_string(status: int) -> str:
    return lib().pbgdn_status_string(int(status)).decode()


def check(status: int, where: str) -> None:
    if status != OK:
        raise PbgdnError(status, where)


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a tensor (None for an absent optional tensor)."""
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream
