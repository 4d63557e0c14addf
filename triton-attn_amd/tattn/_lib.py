"""ctypes binding of libtattn_hip.so (the C ABI in include/tattn.h).

The library is loaded after `import torch`, so its `libamdhip64.so.7` dependency resolves to the
HIP runtime torch already mapped: one runtime instance, so torch's stream handles are valid here.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the library is loaded, see above)

LIB_PATH = Path(__file__).resolve().with_name("libtattn_hip.so")
ABI_VERSION = 2

F16, F32, BF16 = 0, 1, 2
K_FWD, K_BWD_DKDV, K_BWD_DQ = 0, 1, 2
KERNEL_NAMES = {K_FWD: "fwd", K_BWD_DKDV: "bwd_dkdv", K_BWD_DQ: "bwd_dq"}

# Every symbol include/tattn.h declares.
EXPORTS = (
    "tattn_abi_version", "tattn_last_error", "tattn_device_supported", "tattn_fwd",
    "tattn_bwd_preprocess", "tattn_bwd_dkdv", "tattn_bwd_dq", "tattn_bwd", "tattn_bwd_noalloc",
    "tattn_num_configs", "tattn_config_desc", "tattn_pick_config",
)


class TattnConfig(ctypes.Structure):
    _fields_ = [
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("tiles", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("kind", ctypes.c_int32),
        ("ring", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
# Stride arguments (const int64_t[4]) are bound as plain addresses: callers pass a ctypes int64
# array, or the address of four consecutive int64 values inside a larger one (one array per call
# holds every tensor's strides).
_STR4 = ctypes.c_void_p

_SIGS = {
    "tattn_abi_version": (_I, []),
    "tattn_last_error": (ctypes.c_char_p, []),
    "tattn_device_supported": (_I, []),
    "tattn_fwd": (_I, [_P, _P, _P, _P, _P, _STR4, _STR4, _STR4, _STR4, _I64, _I64, _I64, _I64, _I, _I, _F, _I, _P]),
    "tattn_bwd_preprocess": (_I, [_P, _P, _P, _STR4, _I64, _I64, _I64, _I64, _I, _P]),
    "tattn_bwd_dkdv": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _STR4, _I64, _I64, _I64, _I64, _I, _I, _F, _I, _P]),
    "tattn_bwd_dq": (_I, [_P, _P, _P, _P, _P, _P, _P, _STR4, _I64, _I64, _I64, _I64, _I, _I, _F, _I, _P]),
    "tattn_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _STR4, _I64, _I64, _I64, _I64, _I, _I, _F, _I, _P]),
    "tattn_bwd_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _STR4, _I64, _I64, _I64, _I64, _I, _I, _F, _I, _P]),
    "tattn_num_configs": (_I, [_I, _I64, _I]),
    "tattn_config_desc": (_I, [_I, _I64, _I, _I, ctypes.POINTER(TattnConfig)]),
    "tattn_pick_config": (_I, [_I, _I64, _I, _I, _I64]),
}

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


class LibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library; raises LibraryMissing if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryMissing(
                    f"{LIB_PATH} is not built: run `python triton-attn_amd/tattn/_build.py` "
                    "(or __graft_entry__.build()) first"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            got = lib.tattn_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH}: ABI version {got}, expected {ABI_VERSION}")
            _lib = lib
    return _lib


def last_error() -> str:
    msg = load().tattn_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")


def strides4(t: torch.Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


_stride_blocks: dict[tuple, tuple] = {}


def stride_block(*ts: torch.Tensor):
    """One int64 array with the four strides of each tensor, and the address of each tensor's
    four. Arrays are kept per distinct stride tuple (read-only for the library), so repeated
    calls on the same layouts build none."""
    key = tuple(t.stride() for t in ts)
    hit = _stride_blocks.get(key)
    if hit is None:
        if len(_stride_blocks) > 1024:
            _stride_blocks.clear()
        arr = (ctypes.c_int64 * (4 * len(ts)))(*(s for st in key for s in st))
        base = ctypes.addressof(arr)
        hit = _stride_blocks[key] = (arr, [base + 32 * i for i in range(len(ts))])
    return hit


def num_configs(kernel: int, d: int, dtype: int) -> int:
    return load().tattn_num_configs(kernel, d, dtype)


def config_desc(kernel: int, d: int, dtype: int, cid: int) -> dict[str, int]:
    out = TattnConfig()
    check(load().tattn_config_desc(kernel, d, dtype, cid, ctypes.byref(out)), "tattn_config_desc")
    return {"id": cid, "block_m": out.block_m, "block_n": out.block_n, "waves": out.waves,
            "tiles": out.tiles, "lds_bytes": out.lds_bytes, "kind": out.kind, "ring": out.ring}


def pick_config(kernel: int, d: int, dtype: int, causal: bool, n: int) -> int:
    rc = load().tattn_pick_config(kernel, d, dtype, int(causal), n)
    if rc < 0:
        raise RuntimeError(f"tattn_pick_config failed: {last_error()}")
    return rc
