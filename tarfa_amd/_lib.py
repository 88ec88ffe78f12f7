"""Loader for libtmoe.so (the HIP C-ABI library).

``torch`` is imported first: libtmoe's HIP runtime symbols then resolve to the
runtime torch has already mapped, so a process never holds two HIP runtimes
(checked after loading).  A missing library raises -- there is no fallback path.
"""
import ctypes
import os
import re

import torch  # noqa: F401  (must precede the library load, see module docstring)

ABI_VERSION = 2
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtmoe.so")

_c = ctypes
_vp, _i, _u64, _sz, _f, _d = _c.c_void_p, _c.c_int, _c.c_uint64, _c.c_size_t, _c.c_float, _c.c_double

# name -> (restype, argtypes); mirrors include/tmoe.h
SIGNATURES = {
    "tmoe_abi_version": (_i, []),
    "tmoe_strerror": (_c.c_char_p, [_i]),
    "tmoe_workspace_bytes": (_sz, [_i] * 6),
    "tmoe_workspace_status": (_i, [_vp, _vp]),
    "tmoe_fill_bf16": (_i, [_vp, _u64, _u64, _f, _u64, _vp]),
    "tmoe_fill_f32": (_i, [_vp, _u64, _u64, _d, _u64, _vp]),
    "tmoe_router_topk": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "tmoe_topk_renorm_bf16": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "tmoe_dispatch": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tmoe_experts_forward_bf16": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "tmoe_moe_block_bf16": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                 _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tmoe_quantize_int4": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "tmoe_dequant_int4_bf16": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp]),
    "tmoe_experts_forward_int4": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "tmoe_moe_block_int4": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                 _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tmoe_moe_layer_bf16": (_i, [_vp, _i, _vp, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                 _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tmoe_moe_layer_int4": (_i, [_vp, _i, _vp, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                 _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tmoe_moe_block_bf16_noalloc": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                         _vp, _vp, _vp, _vp, _vp, _vp]),
    "tmoe_route_telemetry_bytes": (_sz, [_i, _i, _i]),
    "tmoe_route_record": (_i, [_vp, _i, _i, _i, _vp, _sz, _vp]),
    "tmoe_debug_decode_trace": (_i, [_vp, _sz]),
    "tmoe_dequant_int4_f16": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp]),
    "tmoe_experts_forward_int4_f16rows": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "tmoe_moe_block_int4_f16rows": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                         _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
}

_LIB = None


def _hip_runtimes_mapped():
    try:
        with open("/proc/self/maps") as f:
            maps = f.read()
    except OSError:
        return set()
    return set(re.findall(r"\S*libamdhip64\.so\S*", maps))


def lib():
    """The loaded library (loaded on first use).  Every exported entry point gets its
    argument types from SIGNATURES: an unbound name raises instead of being called with
    ctypes' default int arguments."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m tarfa_amd.build` (no CPU fallback exists)")
    handle = _c.CDLL(LIB_PATH)
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(f"two HIP runtimes mapped in one process: {sorted(runtimes)}")
    # The version first: a library built from older sources may lack entry points named below.
    ver = getattr(handle, "tmoe_abi_version", None)
    if ver is None:
        raise RuntimeError(f"{LIB_PATH} exports no tmoe_abi_version: rebuild with `python -m tarfa_amd.build`")
    ver.restype, ver.argtypes = _i, []
    v = ver()
    if v != ABI_VERSION:
        raise RuntimeError(f"libtmoe ABI {v}, expected {ABI_VERSION}: rebuild with `python -m tarfa_amd.build`")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = res, args
    handle = _Bound(handle)
    _LIB = handle
    return handle


class _Bound:
    """The library handle, restricted to the entry points with declared signatures."""

    def __init__(self, handle):
        self._handle = handle
        for name in SIGNATURES:
            setattr(self, name, getattr(handle, name))

    def __getattr__(self, name):
        raise AttributeError(f"libtmoe entry point {name} has no signature in tarfa_amd._lib.SIGNATURES")


def check(status, what):
    """Raise RuntimeError for a non-zero tmoe status."""
    if status != 0:
        msg = lib().tmoe_strerror(status).decode()
        raise RuntimeError(f"{what}: tmoe status {status} ({msg})")


def exported_symbols():
    return sorted(SIGNATURES)
