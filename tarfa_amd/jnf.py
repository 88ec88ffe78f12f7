"""JNF v1, the reference's on-disk execution format for exact-BF16 experts, and the host tier
it feeds.

Layout (format/JNF_V1.md:7-31, written by format/convert_jnf.py:53-87):

    <root>/manifest.json                       format, version, dtype, alignment, router_top_k,
                                               model_id, revision, tokenizer_revision, layers
    <root>/layers/NN/gate_up.bf16              E expert projections [2I, H] bf16, back to back
    <root>/layers/NN/down.bf16                 E expert projections [H, I] bf16
    <root>/layers/NN/index.json                per-projection expert_bytes and offsets

Invariants checked on open (JNF_V1.md:19-31): format "JNF", version 1, dtype BF16, every
expert projection a whole number of 4096-byte blocks at offset e * expert_bytes, explicit
shapes and offsets, SHA-256 for every expert projection and every file; unknown versions,
shapes or failed checksums are refused (``JnfError``).

``JnfModel.read_experts`` is the analogue of the reference's transport
(tarfa/engine/exact_bf16.py:126-193 read_bf16 / _read_bf16_pinned): parallel preads of whole
expert projections straight into pinned host buffers, optionally checking each expert's
SHA-256 as it arrives.  ``tarfa_amd.residency.ResidencyLedger.load_jnf`` fills the ledger from
it: HBM slabs through double-buffered pinned staging and copies on a side stream, or, in the
tiered mode, the pinned host tier itself (the kernels read non-resident experts there until
``promote`` copies them into HBM slots on the side stream).

``write_jnf`` / ``convert_safetensors`` produce the format (atomic per layer: ``.partial`` then
rename, convert_jnf.py:64-72), from tensors or from checkpoint shards holding
``model.layers.N.mlp.experts.gate_up_proj`` / ``down_proj`` (exact_bf16.py:77-89).
"""
import concurrent.futures as cf
import hashlib
import json
import os
import re
import struct

import torch

FORMAT, VERSION, DTYPE, ALIGN = "JNF", 1, "BF16", 4096
PROJ = ("gate_up_proj", "down_proj")
FILE = {"gate_up_proj": "gate_up.bf16", "down_proj": "down.bf16"}
INDEX_KEY = {"gate_up_proj": "gate_up", "down_proj": "down"}
MANDATORY = ("format", "version", "dtype", "alignment", "router_top_k", "model_id", "revision",
             "tokenizer_revision", "layers")
READ_THREADS = 16


class JnfError(ValueError):
    """A JNF tree that the runtime refuses (JNF_V1.md:31)."""


def _sha256(buf):
    return hashlib.sha256(buf).hexdigest()


class JnfLayer:
    """One layer's two projection files: shapes, per-expert byte ranges and hashes."""

    def __init__(self, root, layer, rec, index):
        self.layer = layer
        self.files, self.shapes, self.expert_bytes, self.expert_sha, self.file_sha = {}, {}, {}, {}, {}
        for name in PROJ:
            if name not in rec:
                raise JnfError(f"layer {layer}: {name} missing from the manifest")
            r = rec[name]
            shape = tuple(int(v) for v in r["shape"])
            if len(shape) != 3:
                raise JnfError(f"layer {layer} {name}: shape {shape} is not [E, rows, cols]")
            nb = int(r["expert_bytes"])
            if nb != shape[1] * shape[2] * 2 or nb % ALIGN:
                raise JnfError(f"layer {layer} {name}: expert_bytes {nb} is not a {ALIGN}-aligned {shape[1:]} bf16")
            hashes = list(r["expert_sha256"])
            if len(hashes) != shape[0]:
                raise JnfError(f"layer {layer} {name}: {len(hashes)} expert hashes for {shape[0]} experts")
            ix = index.get(INDEX_KEY[name], {})
            if int(ix.get("expert_bytes", -1)) != nb or [int(o) for o in ix.get("offsets", [])] != \
                    [e * nb for e in range(shape[0])]:
                raise JnfError(f"layer {layer} {name}: index.json offsets are not e * {nb}")
            path = os.path.join(root, r["file"])
            if not os.path.isfile(path) or os.path.getsize(path) != shape[0] * nb:
                raise JnfError(f"layer {layer} {name}: {path} does not hold {shape[0]} x {nb} bytes")
            self.files[name], self.shapes[name], self.expert_bytes[name] = path, shape, nb
            self.expert_sha[name], self.file_sha[name] = hashes, r["file_sha256"]
        g, d = self.shapes["gate_up_proj"], self.shapes["down_proj"]
        if g[0] != d[0] or g[1] != 2 * d[2] or g[2] != d[1]:
            raise JnfError(f"layer {layer}: gate_up {g} and down {d} are not [E, 2I, H] and [E, H, I]")
        self.num_experts, self.hidden, self.intermediate = g[0], g[2], d[2]


class JnfModel:
    """A validated JNF v1 tree.  ``shape`` (a MoEShape), when given, must match every layer."""

    def __init__(self, root, shape=None):
        self.root = os.fspath(root)
        mpath = os.path.join(self.root, "manifest.json")
        try:
            with open(mpath) as f:
                man = json.load(f)
        except (OSError, json.JSONDecodeError) as e:
            raise JnfError(f"{mpath}: {e}") from e
        missing = [k for k in MANDATORY if k not in man]
        if missing:
            raise JnfError(f"manifest lacks mandatory fields {missing}")
        if man["format"] != FORMAT or man["version"] != VERSION:
            raise JnfError(f"unknown format {man['format']!r} version {man['version']!r} (runtime reads JNF 1)")
        if man["dtype"] != DTYPE or int(man["alignment"]) != ALIGN:
            raise JnfError(f"dtype {man['dtype']} / alignment {man['alignment']} (expects BF16 / {ALIGN})")
        self.manifest = man
        self.top_k = int(man["router_top_k"])
        self.layers = {}
        for key, rec in man["layers"].items():
            l = int(key)
            ipath = os.path.join(self.root, "layers", f"{l:02d}", "index.json")
            try:
                with open(ipath) as f:
                    index = json.load(f)
            except (OSError, json.JSONDecodeError) as e:
                raise JnfError(f"{ipath}: {e}") from e
            if int(index.get("layer", -1)) != l:
                raise JnfError(f"{ipath}: names layer {index.get('layer')}")
            self.layers[l] = JnfLayer(self.root, l, rec, index)
        if shape is not None:
            for l, ly in self.layers.items():
                if (ly.num_experts, ly.hidden, ly.intermediate) != (shape.num_experts, shape.hidden,
                                                                    shape.intermediate):
                    raise JnfError(f"layer {l}: E={ly.num_experts} H={ly.hidden} I={ly.intermediate} "
                                   f"does not match {shape}")
            if self.top_k != shape.top_k:
                raise JnfError(f"router_top_k {self.top_k} does not match {shape.top_k}")

    # ------------------------------------------------------------------ reads
    def read_experts(self, layer, experts, gate_up_out, down_out, verify=True, threads=READ_THREADS):
        """Read experts ``experts`` of ``layer`` into host tensors: gate_up_out[j] / down_out[j]
        (bf16 [2I, H] / [H, I] rows, e.g. pinned) receive expert experts[j].  One pread per
        expert projection, ``threads`` at a time (exact_bf16.py:163-175); with ``verify``
        every expert's SHA-256 is checked against the manifest before returning."""
        ly = self.layers[layer]
        experts = [int(e) for e in experts]
        for e in experts:
            if not 0 <= e < ly.num_experts:
                raise IndexError(f"expert {e} outside [0, {ly.num_experts})")
        fds = {name: os.open(ly.files[name], os.O_RDONLY) for name in PROJ}
        try:
            def one(job):
                name, j, e = job
                dst = (gate_up_out if name == "gate_up_proj" else down_out)[j]
                nb = ly.expert_bytes[name]
                if dst.numel() * dst.element_size() != nb or not dst.is_contiguous():
                    raise ValueError(f"{name} destination {j} is not {nb} contiguous bytes")
                mv = memoryview(dst.view(torch.uint8).numpy()).cast("B")
                done = 0
                while done < nb:
                    n = os.preadv(fds[name], [mv[done:]], e * nb + done)
                    if n <= 0:
                        raise JnfError(f"{ly.files[name]}: short read of expert {e}")
                    done += n
                if verify and _sha256(mv) != ly.expert_sha[name][e]:
                    raise JnfError(f"layer {layer} {name} expert {e}: SHA-256 mismatch")
                return nb

            jobs = [(name, j, e) for j, e in enumerate(experts) for name in PROJ]
            with cf.ThreadPoolExecutor(max_workers=max(1, min(threads, len(jobs)))) as ex:
                return sum(ex.map(one, jobs))
        finally:
            for fd in fds.values():
                os.close(fd)

    def verify(self, layer, files=True):
        """Check every expert hash of ``layer`` (and, with ``files``, each whole-file hash)."""
        ly = self.layers[layer]
        for name in PROJ:
            nb, whole = ly.expert_bytes[name], hashlib.sha256()
            with open(ly.files[name], "rb") as f:
                for e in range(ly.num_experts):
                    blk = f.read(nb)
                    if _sha256(blk) != ly.expert_sha[name][e]:
                        raise JnfError(f"layer {layer} {name} expert {e}: SHA-256 mismatch")
                    whole.update(blk)
            if files and whole.hexdigest() != ly.file_sha[name]:
                raise JnfError(f"layer {layer} {name}: file SHA-256 mismatch")


# ------------------------------------------------------------------ writing
def _write_projection(path, chunks):
    """Write ``chunks`` (bytes-likes, one per expert) to path.partial, then rename; returns
    (file hash, per-expert hashes)."""
    whole, hashes = hashlib.sha256(), []
    tmp = path + ".partial"
    with open(tmp, "wb", buffering=0) as f:
        for c in chunks:
            mv = memoryview(c).cast("B")
            f.write(mv)
            whole.update(mv)
            hashes.append(_sha256(mv))
    os.replace(tmp, path)
    return whole.hexdigest(), hashes


def _finish(root, records, top_k, model_id, revision, tokenizer_revision, old=None):
    man = {"format": FORMAT, "version": VERSION, "dtype": DTYPE, "alignment": ALIGN, "router_top_k": int(top_k),
           "model_id": model_id, "revision": revision, "tokenizer_revision": tokenizer_revision,
           "layers": dict(old or {})}
    man["layers"].update({str(l): r for l, r in records.items()})
    tmp = os.path.join(root, "manifest.json.partial")
    with open(tmp, "w") as f:
        json.dump(man, f, indent=1)
    os.replace(tmp, os.path.join(root, "manifest.json"))


def _layer_record(root, layer, sources):
    """sources: name -> (shape, iterator of per-expert bytes-likes)."""
    ld = os.path.join(root, "layers", f"{layer:02d}")
    os.makedirs(ld, exist_ok=True)
    rec = {}
    for name in PROJ:
        shape, chunks = sources[name]
        nb = shape[1] * shape[2] * 2
        if nb % ALIGN:
            raise JnfError(f"layer {layer} {name}: expert bytes {nb} not {ALIGN}-aligned")
        path = os.path.join(ld, FILE[name])
        fh, eh = _write_projection(path, chunks)
        rec[name] = {"file": os.path.relpath(path, root), "shape": list(shape), "expert_bytes": nb,
                     "file_sha256": fh, "expert_sha256": eh}
    idx = {"layer": layer}
    for name in PROJ:
        nb = rec[name]["expert_bytes"]
        idx[INDEX_KEY[name]] = {"expert_bytes": nb, "offsets": [e * nb for e in range(rec[name]["shape"][0])]}
    with open(os.path.join(ld, "index.json"), "w") as f:
        json.dump(idx, f)
    return rec


def _experts_of(host):
    return (host[e].view(torch.uint8).numpy() for e in range(host.shape[0]))


def write_jnf(root, layers, top_k=8, model_id=None, revision=None, tokenizer_revision=None):
    """Write layers {l: (gate_up [E, 2I, H], down [E, H, I]) bf16 tensors, any device} as JNF v1."""
    root = os.fspath(root)
    os.makedirs(root, exist_ok=True)
    old = None
    mpath = os.path.join(root, "manifest.json")
    if os.path.exists(mpath):
        with open(mpath) as f:
            old = json.load(f).get("layers")
    records = {}
    for l, (gu, dn) in sorted(layers.items()):
        src = {}
        for name, t in (("gate_up_proj", gu), ("down_proj", dn)):
            if t.dtype != torch.bfloat16 or t.dim() != 3:
                raise JnfError(f"layer {l} {name}: expects a [E, rows, cols] bf16 tensor")
            host = t.detach().to("cpu").contiguous()
            src[name] = (tuple(host.shape), _experts_of(host))
        records[int(l)] = _layer_record(root, int(l), src)
    _finish(root, records, top_k, model_id, revision, tokenizer_revision, old)


_EXPERT_RE = re.compile(r"layers\.(\d+)\.mlp\.experts\.(gate_up_proj|down_proj)$")


def convert_safetensors(shards, root, layers=None, top_k=8, model_id=None, revision=None,
                        tokenizer_revision=None, verify=True):
    """Build a JNF v1 tree from checkpoint shards holding ``...layers.N.mlp.experts.gate_up_proj``
    [E, 2I, H] and ``down_proj`` [E, H, I] in BF16 (exact_bf16.py:77-89 finds them the same way;
    convert_jnf.py:53-87 writes them).  Experts are streamed one at a time; with ``verify``,
    every emitted region is re-read and compared with its source (convert_jnf.py:89-107)."""
    found = {}
    for sh in shards:
        with open(sh, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            if n > 100_000_000:
                continue
            hdr = json.loads(f.read(n))
        for key, v in hdr.items():
            m = _EXPERT_RE.search(key)
            if not m:
                continue
            if v["dtype"] != "BF16":
                raise JnfError(f"{key}: dtype {v['dtype']} != BF16")
            found.setdefault(int(m.group(1)), {})[m.group(2)] = (os.fspath(sh), 8 + n + v["data_offsets"][0],
                                                                  tuple(v["shape"]))
    todo = sorted(found) if layers is None else [int(l) for l in layers]
    root = os.fspath(root)
    os.makedirs(root, exist_ok=True)

    def stream(path, offset, shape):
        nb = shape[1] * shape[2] * 2
        fd = os.open(path, os.O_RDONLY)
        try:
            for e in range(shape[0]):
                buf = bytearray(nb)
                if os.preadv(fd, [buf], offset + e * nb) != nb:
                    raise JnfError(f"{path}: short read")
                yield buf
        finally:
            os.close(fd)

    records = {}
    for l in todo:
        if set(found.get(l, {})) != set(PROJ):
            raise JnfError(f"layer {l}: expert projections {sorted(found.get(l, {}))} in the shards")
        src = {name: (found[l][name][2], stream(*found[l][name])) for name in PROJ}
        records[l] = _layer_record(root, l, src)
        if verify:
            for name in PROJ:
                path, off, shape = found[l][name]
                emitted = os.path.join(root, records[l][name]["file"])
                with open(emitted, "rb") as a:
                    for e, want in enumerate(stream(path, off, shape)):
                        got = a.read(len(want))
                        if got != bytes(want) or _sha256(got) != records[l][name]["expert_sha256"][e]:
                            raise JnfError(f"layer {l} {name} expert {e}: emitted bytes differ from the source")
    old = None
    mpath = os.path.join(root, "manifest.json")
    if os.path.exists(mpath):
        with open(mpath) as f:
            old = json.load(f).get("layers")
    _finish(root, records, top_k, model_id, revision, tokenizer_revision, old)
    return sorted(records)
