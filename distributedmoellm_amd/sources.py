"""Expert weights read out of checkpoint files through a read-only memory map.

Two container formats, each read from its published byte layout:

safetensors
    ``u64le n | n bytes of UTF-8 JSON | data``. The JSON object maps each
    tensor name to ``{"dtype", "shape", "data_offsets": [begin, end]}`` with
    offsets counted from the first data byte; an optional ``__metadata__``
    entry holds free-form strings. A checkpoint is a directory of one or more
    such files, optionally listed by ``model.safetensors.index.json``
    (``{"weight_map": {tensor: file}}``).

GGUF, versions 2 and 3 (little-endian)
    ``"GGUF" | u32 version | u64 tensor count | u64 key count``, then the
    key/value records (string key, u32 value type, value), then one record per
    tensor (string name, u32 rank, u64 extent per dimension innermost first,
    u32 ggml type, u64 offset), then zero padding up to a multiple of
    ``general.alignment`` (32 when absent). Tensor data starts there; each
    offset is counted from that point and is itself a multiple of the
    alignment. A string is ``u64 length | bytes``; value types 0-7 and 10-12
    are fixed-size scalars, 8 a string, 9 an array (u32 element type, u64
    count, elements).

What the expert path takes from them (the behaviour of moelan's readers:
moelan/safetensors_io.py:45-138, moelan/config.py:70-86 and 185-195,
moelan/experts.py:403-458, moelan/gguf.py:87-171 and 373-402):

- a colibri int4 container is a safetensors checkpoint next to a
  ``qwen36_meta.json`` with ``ebits`` 4 and a group size ``expert_gs``; one
  expert is two tensors, ``merged_weight`` (packed int4 rows of gate, up and
  down, in that order) and ``qs`` (their f32 group scales, same order);
- a Hugging Face checkpoint holds each expert as three float tensors
  (gate, up, down projections), read as f32 experts;
- in a GGUF MoE file expert ``e`` of layer ``L`` is slice ``e`` of the
  stacked tensors ``blk.L.ffn_{gate,up,down}_exps.weight``.

Experts come out as views of the memory map (no copy in host RAM); their
matrices make one device copy on first use, so weights go from the page cache
to HBM in one transfer.
"""

from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import gguf as G
from .experts import Expert, F32Matrix, Packed4


def _map_file(path: Path) -> np.ndarray:
    """The whole file as a read-only uint8 array backed by an mmap (slices of
    a plain ndarray are cheap views, unlike np.memmap's)."""
    with open(path, "rb") as f:
        if os.fstat(f.fileno()).st_size == 0:
            return np.zeros(0, np.uint8)
        return np.frombuffer(mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ), np.uint8)


# ================================================================ safetensors

# the format's dtype tags -> numpy storage type (BF16 is kept as raw 16-bit words)
ST_DTYPES = {"F64": np.dtype("<f8"), "F32": np.dtype("<f4"), "F16": np.dtype("<f2"), "BF16": np.dtype("<u2"),
             "I64": np.dtype("<i8"), "I32": np.dtype("<i4"), "I16": np.dtype("<i2"), "I8": np.dtype("i1"),
             "U8": np.dtype("u1"), "BOOL": np.dtype("?")}


@dataclass(frozen=True)
class Span:
    """Where one tensor's bytes lie in its file (absolute offsets)."""
    dtype: str
    shape: tuple
    start: int
    stop: int

    @property
    def nbytes(self) -> int:
        return self.stop - self.start


def safetensors_index(path) -> tuple[dict[str, Span], dict]:
    """({name: Span}, metadata) of one safetensors file, checked against the
    file's size: every tensor must lie inside the data section, and a tensor
    of a known dtype must hold exactly prod(shape) elements."""
    path = Path(path)
    size = path.stat().st_size
    with open(path, "rb") as f:
        prefix = f.read(8)
        if len(prefix) != 8:
            raise ValueError(f"{path}: too short for a safetensors file")
        hlen = int.from_bytes(prefix, "little")
        if hlen > size - 8:
            raise ValueError(f"{path}: header length {hlen} runs past the end of the file")
        doc = json.loads(f.read(hlen).decode("utf-8"))
    if not isinstance(doc, dict):
        raise ValueError(f"{path}: the header is not a JSON object")
    data0 = 8 + hlen
    metadata = doc.pop("__metadata__", None) or {}
    spans = {}
    for name, d in doc.items():
        lo, hi = (int(v) for v in d["data_offsets"])
        shape = tuple(int(v) for v in d["shape"])
        if not 0 <= lo <= hi or data0 + hi > size:
            raise ValueError(f"{path}: tensor {name!r} ({lo}..{hi}) lies past the end of the file")
        dt = ST_DTYPES.get(d["dtype"])
        if dt is not None and hi - lo != int(np.prod(shape, dtype=np.int64)) * dt.itemsize:
            raise ValueError(f"{path}: tensor {name!r} has {hi - lo} bytes for {d['dtype']}{list(shape)}")
        spans[name] = Span(d["dtype"], shape, data0 + lo, data0 + hi)
    return spans, metadata


def widen(buf: np.ndarray, tag: str, shape, dtype=np.float32) -> np.ndarray:
    """A tensor's bytes as a new array of ``dtype`` (BF16 words widened exactly)."""
    a = np.frombuffer(buf, ST_DTYPES[tag]).reshape(shape)
    if tag == "BF16":
        a = (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(dtype)


class SafetensorsFile:
    """One safetensors file; the data are mapped on first access."""

    def __init__(self, path):
        self.path = Path(path)
        self.spans, self.metadata = safetensors_index(self.path)
        self._bytes = None

    def names(self):
        return self.spans.keys()

    def raw(self, name: str):
        """(uint8 view of the tensor's bytes in the map, dtype tag, shape list)."""
        if self._bytes is None:
            self._bytes = _map_file(self.path)
        sp = self.spans[name]
        return self._bytes[sp.start:sp.stop], sp.dtype, list(sp.shape)

    def get(self, name: str, dtype=np.float32) -> np.ndarray:
        return widen(*self.raw(name), dtype)

    def nbytes(self, name: str) -> int:
        return self.spans[name].nbytes


class Checkpoint:
    """A checkpoint directory of safetensors files: tensor name -> file from
    the index file when there is one, else from the files' own headers."""

    INDEX = "model.safetensors.index.json"

    def __init__(self, root):
        self.root = Path(root)
        self._open: dict[str, SafetensorsFile] = {}
        index = self.root / self.INDEX
        if index.is_file():
            self.file_of = dict(json.loads(index.read_text())["weight_map"])
        else:
            self.file_of = {}
            for p in sorted(self.root.glob("*.safetensors")):
                f = self._open[p.name] = SafetensorsFile(p)
                self.file_of.update(dict.fromkeys(f.names(), p.name))
        if not self.file_of:
            raise FileNotFoundError(f"no safetensors tensors under {self.root}")

    def file(self, name: str) -> SafetensorsFile:
        fname = self.file_of[name]
        f = self._open.get(fname)
        if f is None:
            f = self._open[fname] = SafetensorsFile(self.root / fname)
        return f

    def __contains__(self, name: str) -> bool:
        return name in self.file_of

    def keys(self):
        return self.file_of.keys()

    def raw(self, name: str):
        return self.file(name).raw(name)

    def get(self, name: str, dtype=np.float32) -> np.ndarray:
        return self.file(name).get(name, dtype)

    def nbytes(self, name: str) -> int:
        return self.file(name).nbytes(name)


# ================================================================ model configuration

# model family -> (name of the MoE block in a layer, gate / up / down projection names)
_EXPERT_TENSORS = {"mixtral": ("block_sparse_moe", ("w1", "w3", "w2")),
                   "phimoe": ("block_sparse_moe", ("w1", "w3", "w2"))}
_USUAL_TENSORS = ("mlp", ("gate_proj", "up_proj", "down_proj"))


@dataclass
class ContainerConfig:
    """The part of a model's configuration the expert path reads (the fields
    and ``expert_names`` of moelan/config.py's ModelConfig)."""
    hidden_size: int
    moe_intermediate_size: int
    num_experts: int
    num_layers: int
    expert_layout: str = "hf"     # "colibri_int4", "gguf" or "hf" (float tensors)
    expert_gs: int = 0            # int4 scale group of a colibri container
    family: str = "qwen3_moe"
    num_experts_per_tok: int = 8

    @property
    def top_k(self) -> int:
        return self.num_experts_per_tok

    def expert_names(self, layer: int, expert: int) -> tuple[str, ...]:
        """One routed expert's tensors: (merged weight, scales) in a colibri
        container, else its (gate, up, down) projections."""
        block, projections = _EXPERT_TENSORS.get(self.family, _USUAL_TENSORS)
        stem = f"model.layers.{layer}.{block}.experts.{expert}."
        if self.expert_layout == "colibri_int4":
            return stem + "merged_weight", stem + "qs"
        return tuple(f"{stem}{p}.weight" for p in projections)


def load_config(model_dir) -> ContainerConfig:
    """A checkpoint's config.json, with the colibri marker file when present."""
    d = Path(model_dir)
    c = json.loads((d / "config.json").read_text())
    c = c.get("text_config", c) if "hidden_size" not in c else c
    first = lambda *keys: next(c[k] for k in keys if c.get(k))  # noqa: E731
    cfg = ContainerConfig(hidden_size=int(c["hidden_size"]),
                          moe_intermediate_size=int(first("moe_intermediate_size", "intermediate_size")),
                          num_experts=int(first("num_experts", "num_local_experts")),
                          num_layers=int(c["num_hidden_layers"]), family=str(c.get("model_type", "qwen3_moe")),
                          num_experts_per_tok=int(c.get("num_experts_per_tok") or 8))
    marker = d / "qwen36_meta.json"
    if marker.is_file():
        m = json.loads(marker.read_text())
        if m.get("ebits") != 4:
            raise ValueError(f"colibri container with ebits={m.get('ebits')} is not supported (int4 only)")
        if not m.get("expert_gs"):
            raise ValueError("colibri container without group scales (expert_gs) is not supported")
        cfg.expert_layout, cfg.expert_gs = "colibri_int4", int(m["expert_gs"])
    return cfg


# ================================================================ checkpoint experts

def colibri_expert(merged, scales, H: int, I: int, gs: int) -> Expert:
    """Split one colibri expert. ``merged`` holds 3*I*H/2 bytes: the 2*I rows of
    gate and up ([2I, H/2]) then the H rows of down ([H, I/2]); ``scales`` the
    f32 group scales in the same row order ([2I, H/gs] then [H, I/gs]). The
    matrices are views of the arguments."""
    merged, scales = np.asarray(merged).reshape(-1), np.asarray(scales).reshape(-1)
    cut_b, cut_s = I * H, 2 * I * H // gs           # where down starts, in bytes and in scales
    if merged.size != cut_b + H * I // 2 or scales.size != cut_s + H * I // gs:
        raise ValueError(f"an expert of {merged.size} bytes and {scales.size} scales does not fit "
                         f"H={H}, I={I}, gs={gs}")
    gu = Packed4(merged[:cut_b].reshape(2 * I, H // 2), scales[:cut_s].reshape(2 * I, H // gs), gs, (2 * I, H))
    down = Packed4(merged[cut_b:].reshape(H, I // 2), scales[cut_s:].reshape(H, I // gs), gs, (H, I))
    return Expert(gu, down, I)


def float_expert(gate, up, down, I: int) -> Expert:
    """An f32 expert from its three float projections ([I, H], [I, H], [H, I])."""
    return Expert(F32Matrix(np.concatenate([gate, up], 0)), F32Matrix(down), I)


def build_expert(cfg, get) -> Expert:
    """The expert whose tensors ``get(part)`` returns: parts "w" and "qs" of a
    colibri container, else "gate", "up" and "down" as f32 arrays."""
    H, I = int(cfg.hidden_size), int(cfg.moe_intermediate_size)
    if cfg.expert_layout == "colibri_int4":
        return colibri_expert(get("w"), get("qs"), H, I, int(cfg.expert_gs))
    return float_expert(get("gate"), get("up"), get("down"), I)


class CheckpointSource:
    """Experts straight out of a safetensors checkpoint. Colibri int4 experts
    are views of the memory map (``zero_copy``); float experts are read into
    f32 arrays. ``cfg``: any object with the fields of :class:`ContainerConfig`
    and its ``expert_names`` (moelan's ModelConfig is one); read from the
    directory when omitted."""

    def __init__(self, model_dir, cfg=None):
        self.cfg = cfg if cfg is not None else load_config(model_dir)
        self.st = Checkpoint(model_dir)
        self.zero_copy = self.cfg.expert_layout == "colibri_int4"
        self._parts = ("w", "qs") if self.zero_copy else ("gate", "up", "down")

    def has(self, key) -> bool:
        return self.cfg.expert_names(*key)[0] in self.st

    def _tensor(self, name: str):
        view, tag, shape = self.st.raw(name)
        if not self.zero_copy:
            return widen(view, tag, shape)
        if tag == "U8":
            return view
        if tag == "F32":
            return view.view(np.float32).reshape(shape)
        raise ValueError(f"{name}: dtype {tag} in a colibri container (U8 weights and F32 scales expected)")

    def load(self, key) -> Expert:
        tensors = dict(zip(self._parts, self.cfg.expert_names(*key)))
        return build_expert(self.cfg, lambda part: self._tensor(tensors[part]))

    def nbytes(self, key) -> int:
        return sum(self.st.nbytes(n) for n in self.cfg.expert_names(*key))


# ================================================================ GGUF

class _Fields:
    """Reads little-endian fields one after another from a byte buffer,
    raising ValueError at the first field that would run past its end."""

    # GGUF value types of fixed size -> struct format
    SCALARS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
    STRING, ARRAY = 8, 9

    def __init__(self, buf, where: str):
        self.buf, self.pos, self.where = buf, 0, where
        self._st = {t: struct.Struct("<" + c) for t, c in self.SCALARS.items()}

    def _need(self, n: int) -> None:
        if self.pos + n > len(self.buf):
            raise ValueError(f"{self.where}: header truncated at byte {self.pos}")

    def scalar(self, vtype: int):
        st = self._st[vtype]
        self._need(st.size)
        (v,) = st.unpack_from(self.buf, self.pos)
        self.pos += st.size
        return v

    def u32(self) -> int:
        return self.scalar(4)

    def u64(self) -> int:
        return self.scalar(10)

    def string(self) -> str:
        n = self.u64()
        self._need(n)
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s

    def value(self, vtype: int):
        if vtype in self._st:
            return self.scalar(vtype)
        if vtype == self.STRING:
            return self.string()
        if vtype == self.ARRAY:
            etype, count = self.u32(), self.u64()
            if etype in self._st and etype != 7:      # numbers: one numpy read
                dt = np.dtype("<" + self.SCALARS[etype])
                self._need(count * dt.itemsize)
                a = np.frombuffer(self.buf, dt, count, self.pos).copy()
                self.pos += count * dt.itemsize
                return a
            return [self.value(etype) for _ in range(count)]
        raise ValueError(f"{self.where}: unknown GGUF value type {vtype} at byte {self.pos}")


@dataclass
class GGUFTensor:
    """One tensor of a GGUF file: ggml type, numpy-order shape, and its bytes'
    place in the mapped file (absolute offset)."""
    name: str
    qtype: int
    shape: tuple
    start: int
    nbytes: int
    file: "GGUFFile"

    @property
    def type_name(self) -> str:
        return G.QTYPES[self.qtype][0]

    def raw(self) -> np.ndarray:
        """The bytes as (leading dims..., bytes per row) uint8, a view of the map."""
        _, per_block, block_bytes = G.QTYPES[self.qtype]
        row = self.shape[-1] // per_block * block_bytes
        return self.file.bytes[self.start:self.start + self.nbytes].reshape(*self.shape[:-1], row)


class GGUFFile:
    """A GGUF file's metadata (``meta``) and tensor table (``tensors``), over a
    read-only map of the file. Only little-endian files of version 2 or 3 and
    the ggml types of the quantized-matrix table are read."""

    MAGIC = b"GGUF"

    def __init__(self, path):
        self.path = Path(path)
        self.bytes = _map_file(self.path)
        rd = _Fields(self.bytes, str(self.path))
        if bytes(self.bytes[:4]) != self.MAGIC:
            raise ValueError(f"{self.path}: not a GGUF file")
        rd.pos = 4
        self.version = rd.u32()
        if self.version not in (2, 3):
            swapped = int.from_bytes(self.version.to_bytes(4, "little"), "big")
            why = "big-endian files" if swapped in (2, 3) else f"version {self.version}"
            raise ValueError(f"{self.path}: GGUF {why} not supported")
        n_tensors, n_keys = rd.u64(), rd.u64()
        self.meta = {}
        for _ in range(n_keys):
            key = rd.string()
            self.meta[key] = rd.value(rd.u32())
        records = []
        for _ in range(n_tensors):
            name = rd.string()
            extents = [rd.u64() for _ in range(rd.u32())]
            records.append((name, tuple(reversed(extents)), rd.u32(), rd.u64()))
        self.alignment = int(self.meta.get("general.alignment", 32))
        self.data_start = -(-rd.pos // self.alignment) * self.alignment
        self.tensors: dict[str, GGUFTensor] = {}
        for name, shape, qtype, offset in records:
            self.tensors[name] = self._tensor(name, shape, qtype, offset)

    def _tensor(self, name, shape, qtype, offset) -> GGUFTensor:
        if qtype not in G.QTYPES:
            raise ValueError(f"{self.path}: tensor {name!r} has ggml type {qtype}, which is not supported")
        _, per_block, block_bytes = G.QTYPES[qtype]
        if shape[-1] % per_block:
            raise ValueError(f"{self.path}: tensor {name!r} rows of {shape[-1]} are not whole blocks")
        if offset % self.alignment:
            raise ValueError(f"{self.path}: tensor {name!r} at offset {offset} is not aligned")
        nbytes = int(np.prod(shape[:-1], dtype=np.int64)) * (shape[-1] // per_block) * block_bytes
        start = self.data_start + offset
        if start + nbytes > self.bytes.size:
            raise ValueError(f"{self.path}: tensor {name!r} data runs past the end of the file")
        return GGUFTensor(name, qtype, shape, start, nbytes, self)

    def __contains__(self, name) -> bool:
        return name in self.tensors

    def __getitem__(self, name) -> GGUFTensor:
        return self.tensors[name]


_GGUF_OPEN: dict[str, GGUFFile] = {}


def open_gguf(path) -> GGUFFile:
    """The process's one GGUFFile for a path (each file is mapped once)."""
    key = os.path.realpath(path)
    if key not in _GGUF_OPEN:
        _GGUF_OPEN[key] = GGUFFile(key)
    return _GGUF_OPEN[key]


def is_gguf(path) -> bool:
    p = Path(path)
    if not p.is_file():
        return False
    with open(p, "rb") as f:
        return f.read(4) == GGUFFile.MAGIC


def _stack_name(layer: int, part: str) -> str:
    return f"blk.{layer}.ffn_{part}_exps.weight"


def gguf_config(path) -> ContainerConfig:
    """The expert shape of a GGUF MoE model from the architecture's metadata
    keys (``<arch>.embedding_length``, ``.expert_count``, ``.block_count``,
    ``.expert_feed_forward_length``, the latter read off layer 0's stacked gate
    tensor when absent)."""
    g = open_gguf(path)
    arch = g.meta.get("general.architecture")
    md = {k[len(arch) + 1:]: v for k, v in g.meta.items() if arch and k.startswith(arch + ".")}
    if not md.get("expert_count"):
        raise ValueError(f"{path}: not a mixture-of-experts model (no {arch}.expert_count)")
    inter = md.get("expert_feed_forward_length")
    if not inter:
        gate = _stack_name(0, "gate")
        inter = g[gate].shape[1] if gate in g else md.get("feed_forward_length")
    return ContainerConfig(hidden_size=int(md["embedding_length"]), moe_intermediate_size=int(inter),
                           num_experts=int(md["expert_count"]), num_layers=int(md["block_count"]),
                           expert_layout="gguf", family=str(arch),
                           num_experts_per_tok=int(md.get("expert_used_count") or 8))


class GGUFSource:
    """Experts straight out of a GGUF file: expert e of layer L is slice e of
    the layer's three stacked expert tensors, kept in its quantized blocks as
    a view of the map. ``cfg`` as for :class:`CheckpointSource`, read from the
    file's metadata when omitted."""

    zero_copy = True
    PARTS = ("gate", "up", "down")

    def __init__(self, path, cfg=None):
        self.g = open_gguf(path)
        self.cfg = cfg if cfg is not None else gguf_config(path)
        self._stacks: dict[int, tuple | None] = {}

    def _layer(self, layer: int):
        """The layer's (gate, up, down) stacked tensors, or None."""
        if layer not in self._stacks:
            names = [_stack_name(layer, p) for p in self.PARTS]
            self._stacks[layer] = tuple(self.g[n] for n in names) if all(n in self.g for n in names) else None
        return self._stacks[layer]

    def has(self, key) -> bool:
        stacks = self._layer(key[0])
        return stacks is not None and 0 <= key[1] < min(self.cfg.num_experts, stacks[0].shape[0])

    def load(self, key) -> Expert:
        layer, e = key
        mats = []
        for t in self._layer(layer):
            if t.qtype not in G.QUANTIZED:
                raise ValueError(f"{t.name}: {t.type_name} experts are not on the device path "
                                 f"(quantized types only)")
            mats.append(G.QuantMatrix(t.raw()[e], t.qtype, t.shape[-1]))
        gate, up, down = mats
        return Expert(G.Stacked(gate, up), down, int(self.cfg.moe_intermediate_size))

    def nbytes(self, key) -> int:
        return sum(t.nbytes // t.shape[0] for t in self._layer(key[0]))


def open_source(model_dir, cfg=None):
    """Where experts are read from: a GGUF file, or a checkpoint directory
    (moelan/experts.py:304-309's ``open_source(model_dir, cfg)``)."""
    if (cfg is not None and getattr(cfg, "expert_layout", None) == "gguf") or is_gguf(model_dir):
        return GGUFSource(model_dir, cfg)
    return CheckpointSource(model_dir, cfg)


__all__ = ["ST_DTYPES", "Span", "safetensors_index", "widen", "SafetensorsFile", "Checkpoint", "ContainerConfig",
           "load_config", "colibri_expert", "float_expert", "build_expert", "CheckpointSource", "GGUFTensor",
           "GGUFFile", "open_gguf", "is_gguf", "gguf_config", "GGUFSource", "open_source"]
