"""Checkpoint files to experts (moelan/safetensors_io.py, moelan/config.py:
185-195, moelan/experts.py:403-458 and 538-639, moelan/gguf.py:87-171 and
373-402), without a GPU: the readers return exactly the bytes a writer put
in the files (written here by the safetensors library and by a GGUF writer
built from the format's published layout), as views of the memory map, and
the store's tiers count and evict as the reference's."""

import json
import struct

import numpy as np
import pytest

from distributedmoellm_amd import experts as X
from distributedmoellm_amd import gguf as G
from distributedmoellm_amd import sources as S

safetensors_numpy = pytest.importorskip("safetensors.numpy")


# ---------------------------------------------------------------- writers

def write_colibri(root, H=256, I=128, gs=64, layers=2, experts=4, seed=0, shards=1):
    """A colibri int4 container: config.json, qwen36_meta.json and
    merged_weight (gate | up | down packed bytes) + qs (f32 scales) per expert.
    Returns {(layer, expert): (bytes, scales)} as written."""
    rng = np.random.default_rng(seed)
    root.mkdir(parents=True, exist_ok=True)
    (root / "config.json").write_text(json.dumps({
        "model_type": "qwen3_moe", "hidden_size": H, "moe_intermediate_size": I, "num_experts": experts,
        "num_hidden_layers": layers, "num_experts_per_tok": 2}))
    (root / "qwen36_meta.json").write_text(json.dumps({"model_type": "qwen3_moe", "ebits": 4, "expert_gs": gs,
                                                       "num_experts": experts}))
    written, tensors = {}, [{} for _ in range(shards)]
    for l in range(layers):
        for e in range(experts):
            w = rng.integers(0, 256, 3 * H * I // 2, dtype=np.uint8)
            s = (np.abs(rng.normal(0, 0.02, 3 * H * I // gs)) / 8).astype(np.float32)
            p = f"model.layers.{l}.mlp.experts.{e}"
            tensors[(l * experts + e) % shards].update({f"{p}.merged_weight": w, f"{p}.qs": s})
            written[(l, e)] = (w, s)
    if shards == 1:
        safetensors_numpy.save_file(tensors[0], str(root / "model.safetensors"))
    else:
        where = {}
        for i, t in enumerate(tensors):
            fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            safetensors_numpy.save_file(t, str(root / fname))
            where.update({n: fname for n in t})
        (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": where}))
    return written


def _gguf_string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, meta: dict, tensors: dict, align: int = 32):
    """A GGUF v3 file: magic, version, tensor and key counts, typed key/values,
    tensor infos (name, dimensions innermost first, type, offset), padding to
    the alignment, then each tensor's data at an aligned offset.
    ``tensors``: name -> (qtype, numpy shape, raw bytes)."""
    kv = b""
    for k, v in meta.items():
        kv += _gguf_string(k)
        if isinstance(v, list) and v and isinstance(v[0], str):
            kv += struct.pack("<IIQ", 9, 8, len(v)) + b"".join(_gguf_string(t) for t in v)
        elif isinstance(v, list):
            kv += struct.pack("<IIQ", 9, 5, len(v)) + struct.pack(f"<{len(v)}i", *v)
        elif isinstance(v, bool):
            kv += struct.pack("<I?", 7, v)
        elif isinstance(v, str):
            kv += struct.pack("<I", 8) + _gguf_string(v)
        elif isinstance(v, float):
            kv += struct.pack("<I", 6) + struct.pack("<f", v)
        else:
            kv += struct.pack("<I", 4) + struct.pack("<I", v)
    infos, blobs, off = b"", [], 0
    for name, (qt, shape, raw) in tensors.items():
        dims = list(reversed(shape))
        infos += _gguf_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<I", qt) + struct.pack("<Q", off)
        data = raw.tobytes()
        pad = (-len(data)) % align
        blobs.append(data + b"\0" * pad)
        off += len(data) + pad
    head = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", len(tensors)) + struct.pack("<Q", len(meta)) + kv + infos
    head += b"\0" * ((-len(head)) % align)
    path.write_bytes(head + b"".join(blobs))


def gguf_moe(path, H=256, I=256, E=4, layers=2, types=(12, 13, 14), seed=0):
    """A GGUF MoE file (qwen3moe metadata) with stacked expert tensors of the
    given (gate, up, down) types and an f32 token embedding. Returns the raw
    stacks {(layer, part): (E, rows, row bytes) uint8}."""
    rng = np.random.default_rng(seed)
    meta = {"general.architecture": "qwen3moe", "general.alignment": 32, "qwen3moe.block_count": layers,
            "qwen3moe.embedding_length": H, "qwen3moe.expert_count": E, "qwen3moe.expert_used_count": 2,
            "qwen3moe.expert_feed_forward_length": I, "qwen3moe.attention.layer_norm_rms_epsilon": 1e-6}
    tensors = {"token_embd.weight": (0, (10, H), rng.standard_normal((10, H)).astype(np.float32))}
    stacks = {}
    for l in range(layers):
        for part, qt, (o, i) in zip(("gate", "up", "down"), types, ((I, H), (I, H), (H, I))):
            raw = np.stack([G.random_blocks(o, i, qt, rng, scale=None) for _ in range(E)])
            tensors[f"blk.{l}.ffn_{part}_exps.weight"] = (qt, (E, o, i), raw)
            stacks[(l, part)] = raw
    write_gguf(path, meta, tensors)
    return stacks


# ---------------------------------------------------------------- colibri

@pytest.mark.parametrize("shards", [1, 3])
def test_colibri_container_reads_views_of_the_bytes_written(tmp_path, shards):
    written = write_colibri(tmp_path / "c", shards=shards)
    cfg = S.load_config(tmp_path / "c")
    assert (cfg.expert_layout, cfg.expert_gs, cfg.hidden_size, cfg.moe_intermediate_size) == ("colibri_int4", 64,
                                                                                              256, 128)
    src = S.CheckpointSource(tmp_path / "c")
    assert src.zero_copy and src.has((1, 3)) and not src.has((2, 0)) and not src.has((0, 4))
    H, I = 256, 128
    for key, (w, s) in written.items():
        e = src.load(key)
        assert e.gu.shape == (2 * I, H) and e.down.shape == (H, I) and e.inter == I and not e.gu.offset
        assert np.array_equal(np.asarray(e.gu.raw).reshape(-1), w[:I * H])
        assert np.array_equal(np.asarray(e.down.raw).reshape(-1), w[I * H:])
        assert np.array_equal(np.asarray(e.gu.s).reshape(-1), s[:2 * I * H // 64])
        assert np.array_equal(np.asarray(e.down.s).reshape(-1), s[2 * I * H // 64:])
        assert not e.gu.raw.flags.owndata and not e.gu.raw.flags.writeable    # a view of the map
        assert src.nbytes(key) == w.nbytes + s.nbytes


def test_colibri_needs_int4_with_groups(tmp_path):
    write_colibri(tmp_path / "c")
    meta = tmp_path / "c" / "qwen36_meta.json"
    meta.write_text(json.dumps({"ebits": 8, "expert_gs": 64}))
    with pytest.raises(ValueError, match="ebits=8"):
        S.load_config(tmp_path / "c")
    meta.write_text(json.dumps({"ebits": 4}))
    with pytest.raises(ValueError, match="expert_gs"):
        S.load_config(tmp_path / "c")


# ---------------------------------------------------------------- GGUF

def test_gguf_file_tensor_table_and_expert_views(tmp_path):
    path = tmp_path / "m.gguf"
    stacks = gguf_moe(path)
    assert S.is_gguf(path) and not S.is_gguf(tmp_path)
    g = S.open_gguf(path)
    assert g.version == 3 and g.meta["general.architecture"] == "qwen3moe"
    t = g["blk.1.ffn_down_exps.weight"]
    assert t.shape == (4, 256, 256) and t.type_name == "Q6_K" and t.nbytes == 4 * 256 * 210
    assert np.array_equal(t.raw(), stacks[(1, "down")])
    emb = g["token_embd.weight"]
    assert emb.shape == (10, 256) and emb.qtype == 0
    cfg = S.gguf_config(path)
    assert (cfg.hidden_size, cfg.moe_intermediate_size, cfg.num_experts, cfg.num_layers) == (256, 256, 4, 2)
    src = S.GGUFSource(path)
    assert src.zero_copy and src.has((0, 3)) and not src.has((0, 4)) and not src.has((2, 0))
    e = src.load((1, 2))
    gate, up = e.gu.parts
    assert (gate.qtype, up.qtype, e.down.qtype) == (12, 13, 14)
    assert np.array_equal(gate.raw, stacks[(1, "gate")][2]) and np.array_equal(up.raw, stacks[(1, "up")][2])
    assert np.array_equal(e.down.raw, stacks[(1, "down")][2])
    assert gate.shape == (256, 256) and e.down.shape == (256, 256) and e.inter == 256
    assert not e.down.raw.flags.owndata
    assert src.nbytes((0, 0)) == 256 * 144 + 256 * 176 + 256 * 210


def test_gguf_rejects_what_it_cannot_read(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(ValueError, match="not a GGUF"):
        S.GGUFFile(p)
    path = tmp_path / "t.gguf"
    write_gguf(path, {"general.architecture": "qwen3moe"}, {"w": (12, (4, 256), np.zeros(4 * 144, np.uint8))})
    data = bytearray(path.read_bytes())
    path.write_bytes(bytes(data[:-64]))                        # truncated tensor data
    with pytest.raises(ValueError, match="past the end"):
        S.GGUFFile(path)
    dense = tmp_path / "d.gguf"
    gguf_moe(dense, types=(0, 0, 0))                           # f32 experts
    with pytest.raises(ValueError, match="quantized types only"):
        S.GGUFSource(dense).load((0, 0))


# ---------------------------------------------------------------- the store's tiers

class FakeSource:
    """Counts loads; zero_copy decides the tier (moelan/experts.py:625-633)."""

    def __init__(self, zero_copy, n=8):
        self.zero_copy, self.n, self.loads = zero_copy, n, 0
        self.rng = np.random.default_rng(1)

    def has(self, key):
        return key[0] == 0 and 0 <= key[1] < self.n

    def load(self, key):
        self.loads += 1
        return X.synthetic_expert(64, 32, "int4", 32, self.rng)


def test_store_tiers_count_and_evict_as_the_reference():
    src = FakeSource(zero_copy=True)
    st = X.ExpertStore([src], map_size=2)
    e0 = st.get((0, 0))
    assert st.misses == 1 and st.hits == 0 and list(st.mapped) == [(0, 0)]
    assert st.get((0, 0)) is e0 and st.misses == 2 and src.loads == 1     # mapped: a miss, not a reload
    st.get((0, 1))
    st.get((0, 2))                                                       # evicts (0, 0)
    assert list(st.mapped) == [(0, 1), (0, 2)]
    st.get((0, 0))                                                       # read again, evicts (0, 1)
    assert src.loads == 4 and list(st.mapped) == [(0, 2), (0, 0)]
    assert st.can_serve((0, 7)) and not st.can_serve((1, 0))
    with pytest.raises(KeyError):
        st.get((1, 0))
    st.forget([(0, 0)])
    assert list(st.mapped) == [(0, 2)]

    copy = FakeSource(zero_copy=False)
    st = X.ExpertStore([copy], lru_size=2)
    a = st.get((0, 3))
    assert st.get((0, 3)) is a and st.hits == 1 and st.misses == 1        # LRU: a hit
    st.get((0, 4))
    st.get((0, 3))                                                       # refresh 3
    st.get((0, 5))                                                       # evicts 4
    assert list(st.lru) == [(0, 3), (0, 5)]
    assert st.resident_bytes() == 2 * a.nbytes
    st = X.ExpertStore([FakeSource(zero_copy=False)])                    # lru_size 0 keeps nothing
    st.get((0, 1))
    assert not st.lru and not st.mapped


def test_store_pinned_experts_and_unpinning():
    rng = np.random.default_rng(2)
    ex = {(0, e): X.synthetic_expert(64, 32, "int4", 32, rng) for e in range(3)}
    st = X.ExpertStore(ex)
    assert st.get((0, 1)) is ex[(0, 1)] and st.hits == 1
    st.unpin_all_except([(0, 2)])
    assert list(st.pinned) == [(0, 2)] and not st.can_serve((0, 1))
    with pytest.raises(ValueError, match="int4 residency"):
        X.to_format(X.synthetic_expert(64, 32, "int8", 32, rng), "int4")


# ---------------------------------------------------------------- format edge cases

def test_safetensors_header_is_checked_against_the_file(tmp_path):
    p = tmp_path / "a.safetensors"
    safetensors_numpy.save_file({"x": np.arange(6, dtype=np.float32).reshape(2, 3),
                                 "b": np.array([1, 2], np.uint16).view(np.uint16)}, str(p))
    f = S.SafetensorsFile(p)
    assert np.array_equal(f.get("x"), np.arange(6, dtype=np.float32).reshape(2, 3))
    view, tag, shape = f.raw("x")
    assert tag == "F32" and shape == [2, 3] and view.nbytes == 24 and not view.flags.writeable
    data = p.read_bytes()
    (tmp_path / "short.safetensors").write_bytes(data[:-8])          # the last tensor cut short
    with pytest.raises(ValueError, match="past the end"):
        S.SafetensorsFile(tmp_path / "short.safetensors")
    hlen = int.from_bytes(data[:8], "little")
    (tmp_path / "long.safetensors").write_bytes((10 ** 9).to_bytes(8, "little") + data[8:])
    with pytest.raises(ValueError, match="header length"):
        S.SafetensorsFile(tmp_path / "long.safetensors")
    doc = json.loads(data[8:8 + hlen])
    doc["x"]["shape"] = [2, 4]                                       # 24 bytes cannot hold 2x4 f32
    head = json.dumps(doc).encode()
    (tmp_path / "shape.safetensors").write_bytes(len(head).to_bytes(8, "little") + head + data[8 + hlen:])
    with pytest.raises(ValueError, match="bytes for F32"):
        S.SafetensorsFile(tmp_path / "shape.safetensors")


def test_bf16_tensors_widen_exactly(tmp_path):
    v = np.array([1.0, -2.5, 3.140625, 1e-3], np.float32)
    bits = (v.view(np.uint32) >> 16).astype(np.uint16)
    p = tmp_path / "h.safetensors"
    head = json.dumps({"t": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 8]}}).encode()
    p.write_bytes(len(head).to_bytes(8, "little") + head + bits.tobytes())
    got = S.SafetensorsFile(p).get("t")
    assert np.array_equal(got, (bits.astype(np.uint32) << 16).view(np.float32))


def test_gguf_metadata_values_and_layout_checks(tmp_path):
    path = tmp_path / "m.gguf"
    meta = {"general.architecture": "qwen3moe", "tokenizer.ggml.tokens": ["a", "bc", "<|im_end|>"],
            "qwen3moe.rope.dims": [1, -2, 3], "qwen3moe.flag": True, "qwen3moe.eps": 0.5}
    write_gguf(path, meta, {"w": (8, (2, 64), np.zeros((2, 68), np.uint8))})
    g = S.GGUFFile(path)
    assert g.meta["tokenizer.ggml.tokens"] == ["a", "bc", "<|im_end|>"]
    assert g.meta["qwen3moe.rope.dims"].tolist() == [1, -2, 3] and g.meta["qwen3moe.flag"] is True
    assert g.meta["qwen3moe.eps"] == 0.5 and g.data_start % 32 == 0
    data = bytearray(path.read_bytes())
    big = bytearray(data)
    big[4:8] = (3).to_bytes(4, "big")
    (tmp_path / "be.gguf").write_bytes(bytes(big))
    with pytest.raises(ValueError, match="big-endian"):
        S.GGUFFile(tmp_path / "be.gguf")
    (tmp_path / "cut.gguf").write_bytes(bytes(data[:40]))            # inside the key/value records
    with pytest.raises(ValueError, match="truncated"):
        S.GGUFFile(tmp_path / "cut.gguf")
    odd = tmp_path / "odd.gguf"                                      # a tensor offset off the alignment
    write_gguf(odd, {"general.architecture": "qwen3moe"}, {"a": (8, (1, 32), np.zeros(34, np.uint8)),
                                                           "b": (8, (1, 32), np.zeros(34, np.uint8))}, align=2)
    with pytest.raises(ValueError, match="not aligned"):
        S.GGUFFile(odd)


def test_float_checkpoint_gives_f32_experts(tmp_path):
    """A Hugging Face checkpoint's float experts (Mixtral naming) load as f32
    experts: gate and up stacked, exact bf16 widening."""
    H, I, E = 64, 32, 2
    rng = np.random.default_rng(7)
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "mixtral", "hidden_size": H,
                                                      "intermediate_size": I, "num_local_experts": E,
                                                      "num_hidden_layers": 1, "num_experts_per_tok": 2}))
    t, want = {}, {}
    for e in range(E):
        p = f"model.layers.0.block_sparse_moe.experts.{e}"
        g, u, d = (rng.standard_normal(s).astype(np.float32) for s in ((I, H), (I, H), (H, I)))
        t.update({f"{p}.w1.weight": g, f"{p}.w3.weight": u, f"{p}.w2.weight": d})
        want[e] = (g, u, d)
    safetensors_numpy.save_file(t, str(tmp_path / "model.safetensors"))
    src = S.open_source(tmp_path)
    assert not src.zero_copy and src.cfg.family == "mixtral" and src.cfg.top_k == 2 and src.has((0, 1))
    e = src.load((0, 1))
    g, u, d = want[1]
    assert isinstance(e.gu, X.F32Matrix) and np.array_equal(e.gu.w, np.concatenate([g, u])) and \
        np.array_equal(e.down.w, d) and e.inter == I


def test_sources_take_a_moelan_style_config(tmp_path):
    """open_source(model_dir, cfg) with a config object of moelan's fields."""
    write_colibri(tmp_path / "c", H=256, I=128, gs=64)

    class ModelConfig:                     # the fields moelan/config.py's ModelConfig gives the sources
        hidden_size, moe_intermediate_size, num_experts = 256, 128, 4
        expert_layout, expert_gs = "colibri_int4", 64

        def expert_names(self, layer, expert):
            p = f"model.layers.{layer}.mlp.experts.{expert}"
            return f"{p}.merged_weight", f"{p}.qs"
    src = S.open_source(tmp_path / "c", ModelConfig())
    assert isinstance(src, S.CheckpointSource) and src.zero_copy
    e = src.load((1, 2))
    assert e.gu.shape == (256, 256) and e.down.shape == (256, 128)
    gpath = tmp_path / "m.gguf"
    gguf_moe(gpath)
    cfg = S.gguf_config(gpath)
    assert isinstance(S.open_source(gpath, cfg), S.GGUFSource)


def test_store_takes_the_reference_arguments():
    """ExpertStore(sources, fmt, lru_size, threads, gs, map_size) as moelan's
    callers pass them; fmt "f32" keeps f32 experts, int8 rounds them in
    groups of gs."""
    rng = np.random.default_rng(8)
    w_gu = rng.standard_normal((64, 64)).astype(np.float32)
    w_dn = rng.standard_normal((64, 32)).astype(np.float32)

    class F32Source:
        zero_copy = False

        def has(self, key):
            return key[0] == 0

        def load(self, key):
            return X.Expert(X.F32Matrix(w_gu), X.F32Matrix(w_dn), 32)
    st = X.ExpertStore([F32Source()], fmt="f32", lru_size=4, threads=3, gs=32, map_size=8)
    assert st.threads == 3 and st.gs == 32 and st.fmt == "f32"
    e, _ = st._read_from((0, 2), st.fmt)                  # what pin() holds (the upload needs a GPU)
    assert isinstance(e.gu, X.F32Matrix)
    st8 = X.ExpertStore([F32Source()], fmt="int8", gs=32)
    q = st8._read_from((0, 0), st8.fmt)[0].gu
    assert isinstance(q, X.GroupQuant) and q.gs == 32 and q.s.shape == (64, 2)
    assert np.abs(q.q.astype(np.float32) * np.repeat(q.s, 32, axis=1) - w_gu).max() <= q.s.max() / 2 + 1e-6
    with pytest.raises(ValueError, match="format"):
        X.ExpertStore([], fmt="bf16")
