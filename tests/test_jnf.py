"""JNF v1 (format/JNF_V1.md, format/convert_jnf.py): writing, validation, refusal of bad
trees, verified reads and conversion from checkpoint shards, on the CPU."""
import json
import os

import numpy as np
import pytest
import torch

from tarfa_amd.jnf import JnfError, JnfModel, convert_safetensors, write_jnf
from tarfa_amd.moe import MoEShape

SHAPE = MoEShape(256, 4, 64, 2, 0)   # expert projections of 2 x 64 x 256 x 2 B = 64 KiB and 32 KiB


def _layers(n=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for l in range(n):
        gu = torch.randn(4, 128, 256, generator=g).to(torch.bfloat16)
        dn = torch.randn(4, 256, 64, generator=g).to(torch.bfloat16)
        out[l] = (gu, dn)
    return out


def test_write_then_read_verified(tmp_path):
    layers = _layers()
    write_jnf(tmp_path, layers, top_k=2, model_id="synthetic", revision="r0", tokenizer_revision="t0")
    m = JnfModel(tmp_path, SHAPE)
    assert sorted(m.layers) == [0, 1] and m.top_k == 2
    for l in (0, 1):
        m.verify(l)
        gu = torch.empty(2, 128, 256, dtype=torch.bfloat16)
        dn = torch.empty(2, 256, 64, dtype=torch.bfloat16)
        assert m.read_experts(l, [3, 1], gu, dn) == 2 * (128 * 256 * 2 + 256 * 64 * 2)
        assert torch.equal(gu[0], layers[l][0][3]) and torch.equal(gu[1], layers[l][0][1])
        assert torch.equal(dn[0], layers[l][1][3]) and torch.equal(dn[1], layers[l][1][1])
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert man["format"] == "JNF" and man["version"] == 1 and man["alignment"] == 4096
    idx = json.loads((tmp_path / "layers" / "00" / "index.json").read_text())
    assert idx["gate_up"]["offsets"] == [e * 65536 for e in range(4)]
    assert not list(tmp_path.rglob("*.partial"))


def test_refuses_unknown_versions_shapes_and_bad_bytes(tmp_path):
    write_jnf(tmp_path, _layers(1), top_k=2)
    mpath = tmp_path / "manifest.json"
    good = mpath.read_text()
    man = json.loads(good)
    man["version"] = 2
    mpath.write_text(json.dumps(man))
    with pytest.raises(JnfError, match="version"):
        JnfModel(tmp_path)
    man = json.loads(good)
    del man["tokenizer_revision"]
    mpath.write_text(json.dumps(man))
    with pytest.raises(JnfError, match="mandatory"):
        JnfModel(tmp_path)
    man = json.loads(good)
    man["layers"]["0"]["down_proj"]["shape"] = [4, 256, 32]
    mpath.write_text(json.dumps(man))
    with pytest.raises(JnfError):
        JnfModel(tmp_path)
    mpath.write_text(good)
    with pytest.raises(JnfError, match="does not match"):
        JnfModel(tmp_path, MoEShape(256, 8, 64, 2, 0))
    # one flipped byte in expert 2's down projection: the verified read and verify() refuse it
    f = tmp_path / "layers" / "00" / "down.bf16"
    raw = bytearray(f.read_bytes())
    raw[2 * 32768 + 100] ^= 0x01
    f.write_bytes(bytes(raw))
    m = JnfModel(tmp_path)
    gu = torch.empty(1, 128, 256, dtype=torch.bfloat16)
    dn = torch.empty(1, 256, 64, dtype=torch.bfloat16)
    m.read_experts(0, [1], gu, dn)                   # an untouched expert still reads
    with pytest.raises(JnfError, match="expert 2: SHA-256"):
        m.read_experts(0, [2], gu, dn)
    with pytest.raises(JnfError, match="SHA-256"):
        m.verify(0)
    m.read_experts(0, [2], gu, dn, verify=False)     # the unverified transport reads the bytes as they are
    # a truncated file
    f.write_bytes(bytes(raw[:-4096]))
    with pytest.raises(JnfError, match="does not hold"):
        JnfModel(tmp_path)


def test_convert_from_checkpoint_shards(tmp_path):
    from safetensors.torch import save_file
    layers = _layers(3, seed=4)
    save_file({"model.layers.0.mlp.experts.gate_up_proj": layers[0][0],
               "model.layers.0.mlp.experts.down_proj": layers[0][1],
               "model.layers.0.self_attn.q_proj.weight": torch.zeros(8, 8, dtype=torch.bfloat16)},
              tmp_path / "model-00001-of-00002.safetensors")
    save_file({"model.layers.1.mlp.experts.gate_up_proj": layers[1][0],
               "model.layers.1.mlp.experts.down_proj": layers[1][1],
               "model.layers.2.mlp.experts.gate_up_proj": layers[2][0],
               "model.layers.2.mlp.experts.down_proj": layers[2][1]},
              tmp_path / "model-00002-of-00002.safetensors")
    out = tmp_path / "jnf"
    shards = sorted(tmp_path.glob("*.safetensors"))
    assert convert_safetensors(shards, out, top_k=2, model_id="synthetic") == [0, 1, 2]
    m = JnfModel(out, SHAPE)
    for l in range(3):
        m.verify(l)
        gu = torch.empty(4, 128, 256, dtype=torch.bfloat16)
        dn = torch.empty(4, 256, 64, dtype=torch.bfloat16)
        m.read_experts(l, range(4), gu, dn)
        assert torch.equal(gu, layers[l][0]) and torch.equal(dn, layers[l][1])
    # per-layer conversion adds to an existing tree (convert_jnf.py --layers)
    out2 = tmp_path / "jnf2"
    convert_safetensors(shards, out2, layers=[2], top_k=2)
    convert_safetensors(shards, out2, layers=[0], top_k=2)
    assert sorted(JnfModel(out2).layers) == [0, 2]
