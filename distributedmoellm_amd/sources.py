"""Where expert weights come from: checkpoint files, memory-mapped, to HBM.

Mirrors the parts of moelan that put experts on the path:
- ``SafeTensorFile`` / ``SafeTensorDir`` (moelan/safetensors_io.py:45-138):
  memory-mapped reading, raw byte views without copies;
- container detection and expert tensor names (moelan/config.py:70-86,
  185-195): a colibri int4 container is a safetensors checkpoint whose
  ``qwen36_meta.json`` says ``ebits`` 4 and ``expert_gs``; an expert is its
  ``merged_weight`` (gate | up | down packed int4 bytes) and ``qs`` (f32
  scales in the same order);
- ``build_expert`` and ``CheckpointSource`` (moelan/experts.py:403-458);
- ``GGUFFile`` / ``open_gguf`` and ``GGUFSource`` (moelan/gguf.py:87-171,
  373-402): the tensor table of a GGUF file, and expert e of a layer as rows
  e of the stacked ``blk.L.ffn_{gate,up,down}_exps.weight`` tensors.

An expert loaded from a source holds views of the file's memory map (no copy
in RAM); its matrices upload one device copy on first use (or when an
``ExpertStore`` pins them), so a checkpoint goes from the page cache to HBM
in one transfer per expert.
"""

from __future__ import annotations

import json
import mmap
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import gguf as G
from .experts import Expert, Packed4

# safetensors dtype tags -> numpy storage types
_DTYPES = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16, "I64": np.int64,
           "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_}


class SafeTensorFile:
    """One .safetensors file: an 8-byte little-endian header length, a JSON
    header of {name: {dtype, shape, data_offsets}}, then the data; mapped
    read-only on first access."""

    def __init__(self, path):
        self.path = Path(path)
        with open(self.path, "rb") as f:
            (hlen,) = struct.unpack("<Q", f.read(8))
            header = json.loads(f.read(hlen))
        self.metadata = header.pop("__metadata__", None) or {}
        self.entries = header
        self._data_offset = 8 + hlen
        self._mm = None

    def _map(self) -> np.ndarray:
        """The file as a read-only uint8 array over an mmap (plain ndarray
        views: slicing one is cheap, unlike np.memmap's)."""
        if self._mm is None:
            with open(self.path, "rb") as f:
                self._mm = np.frombuffer(mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ), np.uint8)
        return self._mm

    def keys(self):
        return self.entries.keys()

    def dtype_tag(self, name: str) -> str:
        return self.entries[name]["dtype"]

    def nbytes(self, name: str) -> int:
        a, b = self.entries[name]["data_offsets"]
        return b - a

    def raw(self, name: str):
        """(a uint8 view of the tensor's bytes in the map, dtype tag, shape)."""
        e = self.entries[name]
        a, b = e["data_offsets"]
        return self._map()[self._data_offset + a:self._data_offset + b], e["dtype"], list(e["shape"])

    def get(self, name: str, dtype=np.float32) -> np.ndarray:
        buf, tag, shape = self.raw(name)
        arr = np.frombuffer(buf, _DTYPES[tag]).reshape(shape)
        if tag == "BF16":
            arr = (arr.astype(np.uint32) << 16).view(np.float32)
        return np.array(arr, dtype=dtype or arr.dtype)


class SafeTensorDir:
    """A checkpoint directory: one or more .safetensors files, or an index."""

    def __init__(self, root):
        self.root = Path(root)
        self.files: dict[str, SafeTensorFile] = {}
        self.where: dict[str, str] = {}
        index = self.root / "model.safetensors.index.json"
        if index.exists():
            self.where.update(json.loads(index.read_text())["weight_map"])
        else:
            for p in sorted(self.root.glob("*.safetensors")):
                for name in SafeTensorFile(p).keys():
                    self.where[name] = p.name
        if not self.where:
            raise FileNotFoundError(f"no safetensors weights in {self.root}")

    def _file(self, name: str) -> SafeTensorFile:
        fname = self.where[name]
        f = self.files.get(fname)
        if f is None:
            f = self.files[fname] = SafeTensorFile(self.root / fname)
        return f

    def __contains__(self, name: str) -> bool:
        return name in self.where

    def keys(self):
        return self.where.keys()

    def raw(self, name: str):
        return self._file(name).raw(name)

    def get(self, name: str, dtype=np.float32) -> np.ndarray:
        return self._file(name).get(name, dtype)

    def nbytes(self, name: str) -> int:
        return self._file(name).nbytes(name)


# ---------------------------------------------------------------- configuration

@dataclass
class ContainerConfig:
    """What the expert path needs of a model's configuration (moelan/config.py:30-86)."""
    hidden_size: int
    moe_intermediate_size: int
    num_experts: int
    num_layers: int
    expert_layout: str = "hf"     # "colibri_int4", "gguf" or "hf"
    expert_gs: int = 0            # int4 scale group (colibri)
    family: str = "qwen3_moe"

    def _mlp(self, layer: int) -> str:
        if self.family in ("mixtral", "phimoe"):
            return f"model.layers.{layer}.block_sparse_moe"
        return f"model.layers.{layer}.mlp"

    def expert_names(self, layer: int, expert: int) -> tuple[str, ...]:
        """The tensors of one routed expert: a colibri container's merged
        weight and scales, or (gate, up, down)."""
        p = f"{self._mlp(layer)}.experts.{expert}"
        if self.expert_layout == "colibri_int4":
            return f"{p}.merged_weight", f"{p}.qs"
        if self.family in ("mixtral", "phimoe"):
            return f"{p}.w1.weight", f"{p}.w3.weight", f"{p}.w2.weight"
        return f"{p}.gate_proj.weight", f"{p}.up_proj.weight", f"{p}.down_proj.weight"


def load_config(model_dir) -> ContainerConfig:
    """config.json plus the colibri marker (moelan/config.py:185-195)."""
    d = Path(model_dir)
    raw = json.loads((d / "config.json").read_text())
    mt = raw.get("model_type", "qwen3_moe")
    family = "mixtral" if mt == "mixtral" else ("phimoe" if mt == "phimoe" else mt)
    cfg = ContainerConfig(hidden_size=int(raw["hidden_size"]),
                          moe_intermediate_size=int(raw.get("moe_intermediate_size") or raw["intermediate_size"]),
                          num_experts=int(raw.get("num_experts") or raw.get("num_local_experts")),
                          num_layers=int(raw["num_hidden_layers"]), family=family)
    meta = d / "qwen36_meta.json"
    if meta.exists():
        m = json.loads(meta.read_text())
        if m.get("ebits") != 4:
            raise ValueError(f"colibri container with ebits={m.get('ebits')} is not supported (int4 only)")
        gs = int(m.get("expert_gs") or 0)
        if not gs:
            raise ValueError("colibri container without group scales (expert_gs) is not supported")
        cfg.expert_layout, cfg.expert_gs = "colibri_int4", gs
    return cfg


# ---------------------------------------------------------------- colibri containers

def build_expert(cfg: ContainerConfig, get) -> Expert:
    """An Expert from its named tensors (moelan/experts.py:403-416): for a
    colibri container ``w`` holds gate | up | down packed rows and ``qs`` their
    f32 scales, in the same order; both stay views of the memory map."""
    if cfg.expert_layout != "colibri_int4":
        raise ValueError("the device expert path reads int4 colibri containers and GGUF files; "
                         f"layout {cfg.expert_layout!r} has f32 experts")
    H, I, gs = cfg.hidden_size, cfg.moe_intermediate_size, cfg.expert_gs
    raw = np.asarray(get("w")).reshape(-1)
    s = np.asarray(get("qs")).reshape(-1)
    ngu, nsu = 2 * I * H // 2, 2 * I * (H // gs)
    if raw.size != ngu + H * I // 2 or s.size != nsu + H * (I // gs):
        raise ValueError(f"expert tensors of {raw.size} bytes and {s.size} scales do not fit H={H}, I={I}, gs={gs}")
    gu = Packed4(raw[:ngu].reshape(2 * I, H // 2), s[:nsu].reshape(2 * I, H // gs), gs, (2 * I, H))
    down = Packed4(raw[ngu:].reshape(H, I // 2), s[nsu:].reshape(H, I // gs), gs, (H, I))
    return Expert(gu, down, I)


class CheckpointSource:
    """Experts read straight out of a checkpoint (moelan/experts.py:419-458):
    int4 experts are views of the shared memory map, no copy in RAM."""

    def __init__(self, model_dir, cfg: ContainerConfig | None = None):
        self.cfg = cfg or load_config(model_dir)
        self.st = SafeTensorDir(model_dir)
        self.zero_copy = self.cfg.expert_layout == "colibri_int4"

    def has(self, key) -> bool:
        return self.cfg.expert_names(*key)[0] in self.st

    def load(self, key) -> Expert:
        names = dict(zip(("w", "qs"), self.cfg.expert_names(*key)))

        def get(part):
            buf, tag, shape = self.st.raw(names[part])
            if tag == "U8":
                return buf
            if tag == "F32":
                return np.frombuffer(buf, np.float32).reshape(shape)
            raise ValueError(f"{names[part]}: dtype {tag} in a colibri container")
        return build_expert(self.cfg, get)

    def nbytes(self, key) -> int:
        return sum(self.st.nbytes(n) for n in self.cfg.expert_names(*key))


# ---------------------------------------------------------------- GGUF files

_GGUF_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q",
                 12: "<d"}


class GGUFTensor:
    __slots__ = ("name", "qtype", "shape", "offset", "nbytes", "file")

    def __init__(self, name, qtype, shape, offset, nbytes, file):
        self.name, self.qtype, self.shape, self.offset, self.nbytes, self.file = \
            name, qtype, shape, offset, nbytes, file

    @property
    def type_name(self) -> str:
        return G.QTYPES[self.qtype][0]

    def raw(self) -> np.ndarray:
        """(rows..., bytes per row) uint8, a view of the memory map."""
        _, block, size = G.QTYPES[self.qtype]
        row_bytes = self.shape[-1] // block * size
        buf = np.frombuffer(self.file.mm, np.uint8, self.nbytes, self.file.data_start + self.offset)
        return buf.reshape(*self.shape[:-1], row_bytes)


class GGUFFile:
    """The header, metadata and tensor table of a GGUF file (version 2 or 3),
    mapped read-only (moelan/gguf.py:87-157). Shapes are in numpy order (the
    file lists dimensions innermost first)."""

    def __init__(self, path):
        self.path = Path(path)
        self._f = open(self.path, "rb")
        self.mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        pos = 0

        def take(fmt):
            nonlocal pos
            v = struct.unpack_from(fmt, self.mm, pos)[0]
            pos += struct.calcsize(fmt)
            return v

        def string():
            nonlocal pos
            n = take("<Q")
            s = bytes(self.mm[pos:pos + n]).decode("utf-8", errors="replace")
            pos += n
            return s

        def value(t):
            nonlocal pos
            if t == 8:
                return string()
            if t == 9:
                et, n = take("<I"), take("<Q")
                if et in _GGUF_SCALARS and et != 7:
                    dt = np.dtype(_GGUF_SCALARS[et])
                    a = np.frombuffer(self.mm, dt, n, pos).copy()
                    pos += n * dt.itemsize
                    return a
                return [value(et) for _ in range(n)]
            if t not in _GGUF_SCALARS:
                raise ValueError(f"{self.path}: unknown GGUF value type {t}")
            return take(_GGUF_SCALARS[t])

        if take("4s") != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        self.version = take("<I")
        if self.version < 2:
            raise ValueError(f"{path}: GGUF version {self.version} is not supported")
        n_tensors, n_kv = take("<Q"), take("<Q")
        self.meta = {}
        for _ in range(n_kv):
            k = string()
            self.meta[k] = value(take("<I"))
        infos = []
        for _ in range(n_tensors):
            name = string()
            dims = [take("<Q") for _ in range(take("<I"))]
            infos.append((name, dims, take("<I"), take("<Q")))
        align = int(self.meta.get("general.alignment", 32))
        self.data_start = (pos + align - 1) // align * align
        self.tensors: dict[str, GGUFTensor] = {}
        for name, dims, qtype, offset in infos:
            if qtype not in G.QTYPES:
                raise ValueError(f"{name}: GGUF tensor type {qtype} is not supported")
            shape = tuple(int(v) for v in reversed(dims))
            _, block, size = G.QTYPES[qtype]
            nbytes = int(np.prod(shape[:-1], dtype=np.int64)) * (shape[-1] // block) * size
            if self.data_start + offset + nbytes > len(self.mm):
                raise ValueError(f"{name}: tensor data past the end of {self.path}")
            self.tensors[name] = GGUFTensor(name, qtype, shape, offset, nbytes, self)

    def __contains__(self, name) -> bool:
        return name in self.tensors

    def __getitem__(self, name) -> GGUFTensor:
        return self.tensors[name]


_OPEN: dict[str, GGUFFile] = {}


def open_gguf(path) -> GGUFFile:
    """One GGUFFile per path (moelan/gguf.py:160-168)."""
    key = str(Path(path).resolve())
    f = _OPEN.get(key)
    if f is None:
        f = _OPEN[key] = GGUFFile(path)
    return f


def gguf_config(path) -> ContainerConfig:
    """The expert shape of a GGUF MoE file from its metadata (moelan/gguf.py:179-236)."""
    g = open_gguf(path)
    arch = g.meta.get("general.architecture")
    k = lambda name, default=None: g.meta.get(f"{arch}.{name}", default)  # noqa: E731
    if not k("expert_count"):
        raise ValueError(f"{path}: not a mixture-of-experts model (no {arch}.expert_count)")
    gate = "blk.0.ffn_gate_exps.weight"
    inter = int(k("expert_feed_forward_length") or (g[gate].shape[1] if gate in g else k("feed_forward_length")))
    return ContainerConfig(hidden_size=int(k("embedding_length")), moe_intermediate_size=inter,
                           num_experts=int(k("expert_count")), num_layers=int(k("block_count")),
                           expert_layout="gguf", family=str(arch))


class GGUFSource:
    """Experts read straight out of a GGUF file (moelan/gguf.py:373-402):
    expert e of layer L is row e of each stacked expert tensor, a view of the
    memory map."""

    zero_copy = True
    PARTS = ("gate", "up", "down")

    def __init__(self, path, cfg: ContainerConfig | None = None):
        self.g = open_gguf(path)
        self.cfg = cfg or gguf_config(path)

    def _tensor(self, layer, part):
        return self.g.tensors.get(f"blk.{layer}.ffn_{part}_exps.weight")

    def has(self, key) -> bool:
        return self._tensor(key[0], "gate") is not None and 0 <= key[1] < self.cfg.num_experts

    def load(self, key) -> Expert:
        mats = []
        for part in self.PARTS:
            t = self._tensor(key[0], part)
            if t.qtype not in G.QUANTIZED:
                raise ValueError(f"{t.name}: {t.type_name} experts are not on the device path (quantized types only)")
            mats.append(G.QuantMatrix(t.raw()[key[1]], t.qtype, t.shape[-1]))
        return Expert(G.Stacked(mats[0], mats[1]), mats[2], self.cfg.moe_intermediate_size)

    def nbytes(self, key) -> int:
        return sum(self._tensor(key[0], p).nbytes // self.cfg.num_experts for p in self.PARTS)


def is_gguf(path) -> bool:
    p = Path(path)
    if not p.is_file():
        return False
    with open(p, "rb") as f:
        return f.read(4) == b"GGUF"


def open_source(path):
    """A source for a model path: a GGUF file or a checkpoint directory."""
    return GGUFSource(path) if is_gguf(path) else CheckpointSource(path)


__all__ = ["SafeTensorFile", "SafeTensorDir", "ContainerConfig", "load_config", "build_expert",
           "CheckpointSource", "GGUFFile", "GGUFTensor", "open_gguf", "gguf_config", "GGUFSource", "is_gguf",
           "open_source"]
