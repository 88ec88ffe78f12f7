"""The reference's int4 file format (tarfa/engine/channel_q4.py:18, 28-38): header parsing,
validation and per-expert reads, on the CPU with synthetic files."""
import json
import struct

import numpy as np
import pytest
import torch

from tarfa_amd.int4_files import NAMES, Int4LayerFile, write_layer_file


def _layer(E=4, H=256, I=128, seed=0, scale_dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    gq = torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, generator=g)
    gs = (torch.randn(E, 2 * I, generator=g) * 0.02).to(scale_dtype)
    dq = torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, generator=g)
    ds = (torch.randn(E, H, generator=g) * 0.02).to(scale_dtype)
    return gq, gs, dq, ds


def test_header_shapes_and_expert_ranges(tmp_path):
    t = _layer()
    p = tmp_path / "layer_0.safetensors"
    write_layer_file(p, *t)
    f = Int4LayerFile(p)
    assert (f.num_experts, f.hidden, f.intermediate) == (4, 256, 128)
    assert f.expert_bytes() == 256 * 128 + 256 * 2 + 256 * 64 + 256 * 2
    got = f.read_experts([3, 0])
    for e in (3, 0):
        for a, b in zip(got[e], t):
            assert a.dtype == (torch.uint8 if b.dtype == torch.uint8 else torch.float16)
            assert torch.equal(a, b[e])
    with pytest.raises(IndexError):
        f.read_experts([4])


def test_bf16_and_f32_scales_become_fp16_as_the_reference_engine_converts_them(tmp_path):
    for dt in (torch.bfloat16, torch.float32):
        t = _layer(scale_dtype=dt, seed=1)
        p = tmp_path / f"layer_{dt}.safetensors"
        write_layer_file(p, *t)
        got = Int4LayerFile(p).read_experts([2])[2]
        assert got[1].dtype == torch.float16 and torch.equal(got[1], t[1][2].to(torch.float16))
        assert torch.equal(got[3], t[3][2].to(torch.float16))


def test_rejects_malformed_files(tmp_path):
    t = _layer()
    # a missing tensor
    from safetensors.torch import save_file
    p = tmp_path / "missing.safetensors"
    save_file({n: v for n, v in zip(NAMES[:3], t[:3])}, p)
    with pytest.raises(ValueError, match="down_s missing"):
        Int4LayerFile(p)
    # inconsistent shapes (down rows do not match H)
    p = tmp_path / "shape.safetensors"
    save_file(dict(zip(NAMES, (t[0], t[1], t[2][:, :128].contiguous(), t[3]))), p)
    with pytest.raises(ValueError, match="shapes"):
        Int4LayerFile(p)
    # packed tensor stored as a float
    p = tmp_path / "dtype.safetensors"
    save_file(dict(zip(NAMES, (t[0].float(), t[1], t[2], t[3]))), p)
    with pytest.raises(ValueError):
        Int4LayerFile(p)
    # a truncated file
    good = tmp_path / "good.safetensors"
    write_layer_file(good, *t)
    raw = good.read_bytes()
    bad = tmp_path / "trunc.safetensors"
    bad.write_bytes(raw[:-100])
    with pytest.raises(ValueError, match="byte range"):
        Int4LayerFile(bad)
    # a header length that cannot be right
    bad.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ValueError, match="header length"):
        Int4LayerFile(bad)


def test_header_matches_the_reference_reader_arithmetic(tmp_path):
    """The byte ranges agree with channel_q4.py:28-38: data start + e * (o1 - o0) / E."""
    t = _layer(E=3)
    p = tmp_path / "l.safetensors"
    write_layer_file(p, *t)
    raw = p.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    h = json.loads(raw[8:8 + n])
    f = Int4LayerFile(p)
    for name in NAMES:
        o0, o1 = h[name]["data_offsets"]
        start, per, _, _ = f.meta[name]
        assert start == 8 + n + o0 and per == (o1 - o0) // 3
        e = 2
        blob = raw[start + e * per:start + (e + 1) * per]
        want = t[NAMES.index(name)][e].contiguous().view(torch.uint8).numpy().tobytes()
        assert blob == want
