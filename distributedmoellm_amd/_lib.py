"""ctypes binding of libmoehip.so (the C ABI of include/moehip.h).

Only pointers, ints and sizes cross the boundary. Device buffers are torch
tensors on the ROCm device (torch owns the memory); ``stream()`` is torch's
current HIP stream, so the kernels order with the caller's torch work.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_char_p, c_int, c_size_t, c_uint32, c_void_p
from pathlib import Path

# MOEHIP_LIB names another build of the library (e.g. a tuning variant)
LIB_PATH = Path(os.environ.get("MOEHIP_LIB") or Path(__file__).with_name("libmoehip.so"))

MOE_OK, MOE_EINVAL, MOE_EHIP, MOE_EWORKSPACE, MOE_EUNSUPPORTED = 0, 1, 2, 3, 4


class MoeError(RuntimeError):
    """A libmoehip call returned a non-zero status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[moehip {code}] {msg}")
        self.code = code


class Q4Expert(ctypes.Structure):
    """``moe_q4_expert``: one int4 expert's device addresses (include/moehip.h)."""
    _fields_ = [("gu_w", c_void_p), ("gu_s", c_void_p), ("dn_w", c_void_p), ("dn_s", c_void_p),
                ("xor8", c_uint32), ("s_f16", ctypes.c_int32)]


_P, _I, _Z = c_void_p, c_int, c_size_t

# name -> (restype, argtypes); the full exported surface
SIGNATURES = {
    "moe_version": (c_int, []),
    "moe_last_error": (c_char_p, []),
    "moe_device_count": (c_int, []),
    "moe_device_info": (c_int, [_I, c_char_p, _I]),
    "moe_init": (c_int, [_I]),
    "moe_q4_matmul_t": (c_int, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "moe_q8_matmul_t": (c_int, [_P, _I, _P, _P, _I, _I, _I, _I, _P, _P]),
    "moe_gguf_matmul_t": (c_int, [_P, _I, _P, _I, _I, _I, _P, _P]),
    "moe_q4_dequant": (c_int, [_P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "moe_q8_dequant": (c_int, [_P, _P, _I, _I, _I, _I, _P, _P]),
    "moe_gguf_dequant": (c_int, [_P, _I, _I, _I, _P, _P]),
    "moe_silu_mul": (c_int, [_P, _I, _I, _I, _P, _I, _P]),
    "moe_combine": (c_int, [_P, _I, _P, _P, _P, _P, _I, _I, _P, _I, _I, _P]),
    "moe_q4_experts_matvec": (c_int, [_P, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _I, _P]),
    "moe_q4_layer_workspace": (c_size_t, [_I, _I, _I]),
    "moe_router_logits_workspace": (c_size_t, [_I, _I, _I]),
    "moe_router_logits": (c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _Z, _P]),
    "moe_route": (c_int, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "moe_group_by_expert": (c_int, [_P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
    "moe_q4_grouped_ffn_workspace": (c_size_t, [_I, _I, _I]),
    "moe_q4_grouped_ffn": (c_int, [_P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _P, _I, _P, _Z, _P]),
    "moe_prefill_workspace": (c_size_t, [_I, _I, _I, _I, _I]),
    "moe_prefill_layer": (c_int, [_P, _I, _P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _P, _Z, _P]),
    "moe_q4_gemm": (c_int, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "moe_q4_layer": (c_int, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _P, _I,
                             _I, _I, _I, _I, _P, _Z, _P]),
    "moe_q4_layer_noalloc": (c_int, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _P, _I,
                                     _I, _I, _I, _I, _P]),
    "moe_q4_layer_i8_workspace": (c_size_t, [_I, _I, _I, _I]),
    "moe_q4_layer_i8": (c_int, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _P, _I,
                                _I, _I, _I, _I, _P, _Z, _P]),
    "moe_round_q8": (c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _P, _P]),
    "moe_wire_encode": (c_int, [_P, _I, _P, _I, _I, _I, _P, _P, _P]),
    "moe_wire_decode": (c_int, [_P, _P, _I, _I, _I, _P, _P, _I, _P]),
}

_lib = None
_why = ""


def load():
    """The loaded library, or None (``why_not()`` says why)."""
    global _lib, _why
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        _why = f"{LIB_PATH.name} is not built (python -m distributedmoellm_amd.build)"
        return None
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        _why = f"{LIB_PATH.name} does not load: {exc}"
        return None
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    _lib = lib
    return lib


def why_not() -> str:
    return _why


def lib():
    """The library; raises when it is not built or does not load."""
    L = load()
    if L is None:
        raise RuntimeError(_why)
    return L


def last_error() -> str:
    L = load()
    return L.moe_last_error().decode(errors="replace") if L is not None else _why


def check(rc: int) -> None:
    if rc != MOE_OK:
        raise MoeError(rc, last_error())


def call(name: str, *args) -> None:
    """Call an int-status entry point and raise MoeError on failure."""
    check(getattr(lib(), name)(*args))


def device_info(device: int = 0) -> dict:
    buf = ctypes.create_string_buffer(512)
    check(lib().moe_device_info(device, buf, len(buf)))
    name, arch, cus, khz, mem = buf.value.decode().split("|")
    return {"name": name, "arch": arch, "cus": int(cus), "clock_khz": int(khz), "hbm_bytes": int(mem)}
