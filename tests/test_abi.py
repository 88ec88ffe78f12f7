"""The C ABI library loads and exports every entry point include/tmoe.h declares (no GPU calls)."""
import ctypes
import os
import re

from tarfa_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "tmoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmoe_\w+)\s*\(", text)))


def test_header_declares_what_the_loader_binds():
    assert declared() == _lib.exported_symbols()


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(handle, n)]
    assert not missing, missing


def test_abi_version_and_strerror():
    lib = _lib.lib()
    assert lib.tmoe_abi_version() == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8):
        assert lib.tmoe_strerror(code).decode() != "unknown tmoe status"
    assert lib.tmoe_strerror(-99).decode() == "unknown tmoe status"


def test_workspace_sizes_and_shape_validation():
    lib = _lib.lib()
    n1 = lib.tmoe_workspace_bytes(1, 2560, 256, 1024, 8, 1024)
    n4k = lib.tmoe_workspace_bytes(4096, 2560, 256, 1024, 8, 1024)
    assert 0 < n1 < n4k
    assert n4k >= 4096 * 8 * 2560 * 2            # per-assignment expert outputs for the combine
    assert lib.tmoe_workspace_bytes(1, 2561, 256, 1024, 8, 0) == 0      # H % 8
    assert lib.tmoe_workspace_bytes(1, 2560, 256, 1024, 9, 0) > 0
    assert lib.tmoe_workspace_bytes(1, 2560, 4, 1024, 8, 0) == 0        # k > E
    assert lib.tmoe_workspace_bytes(0, 2560, 256, 1024, 8, 0) == 0


def test_entry_points_reject_bad_arguments_without_touching_the_device():
    lib = _lib.lib()
    # NULL pointers and bad shapes are rejected on the host before any launch
    assert lib.tmoe_experts_forward_bf16(None, 1, None, None, None, 2560, 256, 1024, 8, None, None, 0, None) == -1
    assert lib.tmoe_experts_forward_bf16(None, 1, None, None, None, 2561, 256, 1024, 8, None, None, 0, None) == -2
    assert lib.tmoe_moe_block_bf16(None, 1, None, None, None, None, None, None, None, 2560, 256, 1024, 8, 0,
                                   None, None, None, None, None, 0, None) == -1
    assert lib.tmoe_router_topk(None, None, None, 1, 2560, 256, 8, None, None, None, None, None) == -1
    assert lib.tmoe_router_topk(None, None, None, 1, 2560, 256, 17, None, None, None, None, None) == -2
    assert lib.tmoe_dispatch(None, 4, 8, 256, None, None, None, None, 0, None) == -1
    assert lib.tmoe_fill_bf16(None, 16, 1, 1.0, 0, None) == -1
    # int4 entry points: NULLs and unsupported shapes (decode: H, I multiples of 512; prefill: of 128)
    assert lib.tmoe_experts_forward_int4(None, 1, None, None, None, 2560, 256, 1024, 8, None, None, 0, None) == -1
    assert lib.tmoe_moe_block_int4(None, 1, None, None, None, None, None, None, None, 2560, 256, 1024, 8, 0,
                                   None, None, None, None, None, 0, None) == -1
    p = 256   # any non-NULL, 16-byte aligned value: rejected before it is dereferenced
    assert lib.tmoe_experts_forward_int4(p, 2, p, p, p, 2560, 256, 960, 8, p, p, 1 << 30, None) == -2  # I % 128
    assert lib.tmoe_experts_forward_int4(p, 1, p, p, p, 2304, 256, 1024, 8, p, p, 1 << 30, None) == -2
    assert lib.tmoe_moe_block_int4(p, 1, p, None, p, p, p, p, p, 2560, 256, 1024, 8, 512,
                                   p, None, None, None, p, 1 << 30, None) == -2        # Is != I
    assert lib.tmoe_quantize_int4(None, 4, 256, 128, None, None, None) == -1
    assert lib.tmoe_quantize_int4(p, 4, 256, 96, p, p, None) == -2                    # K % G
    assert lib.tmoe_quantize_int4(p, 4, 256, 3, p, p, None) == -2                     # odd G
    assert lib.tmoe_dequant_int4_bf16(p, p, 4, 260, 130, p, None) == -2               # K % 8
    assert lib.tmoe_dequant_int4_bf16(p + 2, p, 4, 256, 128, p, None) == -3           # packed alignment
    # the MoE sublayer entry points: the norm weight is required, out must not alias h, eps >= 0
    for fn in (lib.tmoe_moe_layer_bf16, lib.tmoe_moe_layer_int4):
        assert fn(p, 1, None, 1e-6, p, None, p, None, None, None, None, 2560, 256, 1024, 8, 0,
                  512, None, None, None, p, 1 << 30, None) == -1
        assert fn(p, 1, p, 1e-6, p, None, p, None, None, None, None, 2560, 256, 1024, 8, 0,
                  p, None, None, None, p, 1 << 30, None) == -2                          # out == h
        assert fn(p, 1, p, -1.0, p, None, p, None, None, None, None, 2560, 256, 1024, 8, 0,
                  512, None, None, None, p, 1 << 30, None) == -2                        # eps < 0
        assert fn(p, 1, p + 2, 1e-6, p, None, p, None, None, None, None, 2560, 256, 1024, 8, 0,
                  512, None, None, None, p, 1 << 30, None) == -3                        # ln_w alignment
    # T * k above 524288 (the dispatch's LDS mask)
    assert lib.tmoe_dispatch(p, 65537, 8, 16, p, p, p, p, 1 << 40, None) == -2


def test_debug_trace_switch_checks_alignment_without_touching_the_device():
    lib = _lib.lib()
    assert lib.tmoe_debug_decode_trace(ctypes.c_void_p(0x1003), 4096) == -3   # TMOE_ERR_ALIGN
    assert lib.tmoe_debug_decode_trace(None, 0) == 0
