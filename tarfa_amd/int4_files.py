"""The reference's own int4 expert files: one safetensors file per layer.

Layout (tarfa/engine/channel_q4.py:18 ``_NAMES``, :28-38 ``_q4meta``, :39-82 readers):

    gate_up_q  uint8 [E, 2I, H/2]   packed nibbles, low nibble = even column, value = nibble - 8
    gate_up_s  fp16  [E, 2I]        one scale per row (F16; the reader also takes BF16 / F32)
    down_q     uint8 [E, H, I/2]
    down_s     fp16  [E, H]

The reference reads an expert as four byte ranges, ``data_start + e * bytes_per_expert``
(channel_q4.py:28-38, 43-46), and converts the scales to the engine dtype on load
(``.to(eng.device, eng.dtype)``, channel_q4.py:77-78; fused_int4.py:139-141) -- fp16 in its
production engine, so scales stored as BF16 or F32 are rounded to fp16 here as it would.
The experts then run through libtmoe's per-row int4 entry points
(``tmoe_experts_forward_int4_f16rows``); ``dequant_int4_f16`` reproduces the reference's
``dequant_int4`` bit for bit.

``Int4LayerFile`` parses and validates the header without reading tensor data;
``read_experts`` preads chosen experts (host tensors), ``load`` brings every expert of the
layer into HBM at once through one pinned staging buffer.  ``write_layer_file`` writes the
same format (the reference ships no writer; its files come from outside its repository,
channel_q4.py:6).
"""
import json
import os
import struct

import numpy as np
import torch

NAMES = ("gate_up_q", "gate_up_s", "down_q", "down_s")
DTYPES = {"U8": torch.uint8, "F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32}
_NP = {torch.uint8: np.uint8, torch.float16: np.float16, torch.float32: np.float32}
MAX_HEADER = 100_000_000


class Int4LayerFile:
    """Header and per-expert byte ranges of one layer file (validated on open)."""

    def __init__(self, path):
        self.path = os.fspath(path)
        size = os.path.getsize(self.path)
        with open(self.path, "rb") as f:
            raw = f.read(8)
            if len(raw) != 8:
                raise ValueError(f"{self.path}: not a safetensors file (short header)")
            n = struct.unpack("<Q", raw)[0]
            if n > MAX_HEADER or 8 + n > size:
                raise ValueError(f"{self.path}: header length {n} is not plausible")
            header = json.loads(f.read(n))
        base = 8 + n
        self.meta = {}
        for name in NAMES:
            if name not in header:
                raise ValueError(f"{self.path}: tensor {name} missing (expected {NAMES})")
            t = header[name]
            if t.get("dtype") not in DTYPES:
                raise ValueError(f"{self.path}: {name} has unsupported dtype {t.get('dtype')}")
            dtype = DTYPES[t["dtype"]]
            shape = tuple(int(v) for v in t["shape"])
            o0, o1 = (int(v) for v in t["data_offsets"])
            E = shape[0]
            per = int(np.prod(shape[1:])) * torch.empty((), dtype=dtype).element_size()
            if E < 1 or o1 - o0 != E * per or base + o1 > size:
                raise ValueError(f"{self.path}: {name} byte range [{o0}, {o1}) does not hold {shape} {t['dtype']}")
            self.meta[name] = (base + o0, per, shape[1:], dtype)
        gq, gs, dq, ds = (self.meta[k] for k in NAMES)
        if gq[3] != torch.uint8 or dq[3] != torch.uint8 or gs[3] == torch.uint8 or ds[3] == torch.uint8:
            raise ValueError(f"{self.path}: packed tensors must be U8 and scales floating point")
        self.num_experts = header["gate_up_q"]["shape"][0]
        if any(header[k]["shape"][0] != self.num_experts for k in NAMES):
            raise ValueError(f"{self.path}: tensors disagree on the number of experts")
        two_i, half_h = gq[2]
        self.hidden, self.intermediate = 2 * half_h, two_i // 2
        H, I = self.hidden, self.intermediate
        if two_i % 2 or gs[2] != (two_i,) or dq[2] != (H, I // 2) or ds[2] != (H,):
            raise ValueError(f"{self.path}: shapes {[self.meta[k][2] for k in NAMES]} are not "
                             f"[2I, H/2], [2I], [H, I/2], [H] for one H, I")

    def expert_bytes(self):
        return sum(self.meta[k][1] for k in NAMES)

    def read_experts(self, experts):
        """{e: (gate_up_q, gate_up_s, down_q, down_s)} host tensors of the chosen experts (one
        pread per tensor and expert, channel_q4.py:43-46); scales as fp16."""
        out = {}
        fd = os.open(self.path, os.O_RDONLY)
        try:
            for e in experts:
                if not 0 <= e < self.num_experts:
                    raise IndexError(f"expert {e} outside [0, {self.num_experts})")
                parts = []
                for name in NAMES:
                    start, per, shape, dtype = self.meta[name]
                    buf = bytearray(per)
                    if os.preadv(fd, [buf], start + e * per) != per:
                        raise IOError(f"{self.path}: short read of {name} expert {e}")
                    t = torch.frombuffer(buf, dtype=dtype).reshape(shape)
                    parts.append(t.to(torch.float16) if name.endswith("_s") else t)
                out[e] = tuple(parts)
        finally:
            os.close(fd)
        return out

    def load(self, device):
        """Every expert of the layer in HBM: (gate_up_q [E,2I,H/2] u8, gate_up_s [E,2I] fp16,
        down_q [E,H,I/2] u8, down_s [E,H] fp16).  Each tensor is read with one pread into a
        pinned buffer and copied to the device; scales become fp16 on the device."""
        dev = torch.device(device)
        out = []
        fd = os.open(self.path, os.O_RDONLY)
        try:
            for name in NAMES:
                start, per, shape, dtype = self.meta[name]
                n = per * self.num_experts
                pin = torch.empty(n, dtype=torch.uint8, pin_memory=dev.type == "cuda")
                mv = memoryview(pin.numpy())
                done = 0
                while done < n:
                    got = os.preadv(fd, [mv[done:]], start + done)
                    if got <= 0:
                        raise IOError(f"{self.path}: short read of {name}")
                    done += got
                t = pin.to(dev, non_blocking=True).view(dtype).reshape(self.num_experts, *shape)
                out.append(t.to(torch.float16) if name.endswith("_s") else t)
        finally:
            os.close(fd)
        if dev.type == "cuda":
            torch.cuda.current_stream(dev).synchronize()   # the pinned staging buffers are released next
        return tuple(out)


def write_layer_file(path, gate_up_q, gate_up_s, down_q, down_s):
    """Write one layer in the reference's format (host or device tensors; scales written in
    their own dtype).  Atomic: written to ``path + '.partial'``, then renamed."""
    from safetensors.torch import save_file

    tensors = {}
    for name, t in zip(NAMES, (gate_up_q, gate_up_s, down_q, down_s)):
        tensors[name] = t.detach().to("cpu").contiguous()
    tmp = os.fspath(path) + ".partial"
    save_file(tensors, tmp)
    os.replace(tmp, path)
