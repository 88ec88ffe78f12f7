"""bf16 rounding on numpy arrays (oracle, test infrastructure only).

bf16 is the upper half of an IEEE binary32.  Rounding is round-to-nearest,
ties-to-even on the discarded 16 bits, which is what torch's ``.to(bfloat16)``
does on CPU and GPU (the reference casts with it everywhere, e.g.
``transformers/.../modeling_qwen3_5_moe.py:774`` and implicitly after every
bf16 ``F.linear`` in ``tarfa/engine/fused_int4.py:193-194``).
"""
import numpy as np


def bits(x):
    """fp32 (or fp64, first rounded to fp32) -> bf16 bit patterns (uint16), RNE."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def to_f32(b):
    """bf16 bit patterns (uint16) -> exact fp32 values."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def rnd(x):
    """Round to the nearest bf16 value, returned as fp32 (fp64 input rounds via fp32)."""
    return to_f32(bits(x))
