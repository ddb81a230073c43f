"""ctypes binding of libjanus_moe_hip.so (the C ABI declared in include/janus_moe.h).

torch is imported first so that the library binds to the HIP runtime torch already loaded (both name the same
soname), which is what lets torch's stream handles and device pointers be passed straight through. There is no
fallback: if the library is missing or stale the import of the op fails with the path and the build command.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library shares)

LIBRARY = Path(__file__).resolve().with_name("libjanus_moe_hip.so")
ABI_VERSION = 1
EXPORTS = (
    "janus_moe_last_error", "janus_moe_abi_version",
    "janus_moe_router_prep_bytes", "janus_moe_router_prepare",
    "janus_moe_route_workspace_bytes", "janus_moe_route",
    "janus_moe_align_workspace_bytes", "janus_moe_align",
    "janus_moe_experts_workspace_bytes", "janus_moe_experts",
    "janus_moe_block_workspace_bytes", "janus_moe_block_forward", "janus_moe_block_forward_masked",
    "janus_moe_add_rmsnorm", "janus_moe_block_forward_serve",
    "janus_moe_dequant", "janus_moe_profile_events",
    "janus_moe_experts_nvfp4", "janus_moe_dequant_nvfp4", "janus_moe_device_status",
    "janus_moe_block_forward_noalloc", "janus_moe_block_forward_nvfp4",
    "janus_moe_experts_planned_workspace_bytes", "janus_moe_experts_planned",
)

_p, _i, _z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t


class BlockWeights(ctypes.Structure):
    """janus_moe_block_weights."""
    _fields_ = [
        ("H", _i), ("I", _i), ("E", _i), ("top_k", _i), ("I_s", _i),
        ("router_w", _p), ("router_prep", _p), ("router_bias", _p),
        ("gate_up_q", _p), ("gate_up_s", _p), ("down_q", _p), ("down_s", _p),
        ("sh_gate_up_q", _p), ("sh_gate_up_s", _p), ("sh_down_q", _p), ("sh_down_s", _p),
        ("sh_gate_w", _p),
    ]


class BlockWeightsNvfp4(ctypes.Structure):
    """janus_moe_block_weights_nvfp4."""
    _fields_ = [
        ("H", _i), ("I", _i), ("E", _i), ("top_k", _i), ("I_s", _i),
        ("router_w", _p), ("router_prep", _p), ("router_bias", _p),
        ("gate_up", _p), ("gate_up_scale", _p), ("gate_up_global", _p),
        ("down", _p), ("down_scale", _p), ("down_global", _p),
        ("sh_gate_up", _p), ("sh_gate_up_scale", _p), ("sh_gate_up_global", _p),
        ("sh_down", _p), ("sh_down_scale", _p), ("sh_down_global", _p),
        ("sh_gate_w", _p),
    ]


_SIGNATURES = {
    "janus_moe_last_error": (ctypes.c_char_p, []),
    "janus_moe_abi_version": (_i, []),
    "janus_moe_router_prep_bytes": (_z, [_i, _i]),
    "janus_moe_router_prepare": (_i, [_p, _i, _i, _p, _z, _p]),
    "janus_moe_route_workspace_bytes": (_z, [_i, _i, _i]),
    "janus_moe_route": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _z, _p]),
    "janus_moe_align_workspace_bytes": (_z, [_i, _i, _i]),
    "janus_moe_align": (_i, [_p, _i, _i, _i, _i, _p, _p, _p, _p, _z, _p]),
    "janus_moe_experts_workspace_bytes": (_z, [_i, _i, _i, _i, _i]),
    "janus_moe_experts": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p, _z, _p]),
    "janus_moe_block_workspace_bytes": (_z, [_i, _i, _i, _i, _i, _i]),
    "janus_moe_block_forward": (_i, [ctypes.POINTER(BlockWeights), _p, _i, _p, _p, _p, _p, _z, _p]),
    "janus_moe_block_forward_masked": (_i, [ctypes.POINTER(BlockWeights), _p, _p, _i, _p, _p, _p, _p, _z, _p]),
    "janus_moe_add_rmsnorm": (_i, [_p, _p, _p, ctypes.c_float, _p, _i, _i, _p, _p, _p]),
    "janus_moe_block_forward_serve": (_i, [ctypes.POINTER(BlockWeights), _p, _p, _p, ctypes.c_float, _p,
                                           ctypes.c_float, _p, _p, _i, _p, _p, _p, _p, _p, _z, _p]),
    "janus_moe_dequant": (_i, [_p, _p, ctypes.c_long, _i, _p, _p]),
    "janus_moe_profile_events": (_i, [ctypes.POINTER(_p), _i]),
    "janus_moe_experts_nvfp4": (_i, [_p] * 9 + [_i] * 5 + [_p, _p, _z, _p]),
    "janus_moe_dequant_nvfp4": (_i, [_p, _p, _p, ctypes.c_long, _i, _p, _p]),
    "janus_moe_device_status": (_i, [_p, _i, _p]),
    "janus_moe_block_forward_noalloc": (_i, [ctypes.POINTER(BlockWeights), _p, _p, _i, _p, _p, _p, _p]),
    "janus_moe_block_forward_nvfp4": (_i, [ctypes.POINTER(BlockWeightsNvfp4), _p, _p, _i, _p, _p, _p, _p, _z, _p]),
    "janus_moe_experts_planned_workspace_bytes": (_z, [_i] * 6),
    "janus_moe_experts_planned": (_i, [_i] + [_p] * 11 + [_i] * 6 + [_p, _p, _z, _p]),
}

_handle = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises RuntimeError if it is missing, stale or exports the wrong ABI)."""
    global _handle
    if _handle is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY} is missing: build it with `python -m janus_amd.build` (hipcc, gfx950)")
        handle = ctypes.CDLL(str(LIBRARY))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = restype, argtypes
        if handle.janus_moe_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIBRARY}: ABI {handle.janus_moe_abi_version()} != {ABI_VERSION}; rebuild it")
        _handle = handle
    return _handle


class JanusMoeError(RuntimeError):
    """A C ABI call returned a non-zero status."""


def check(status: int, what: str) -> None:
    if status != 0:
        message = lib().janus_moe_last_error().decode(errors="replace")
        raise JanusMoeError(f"{what} failed (status {status}): {message}")
