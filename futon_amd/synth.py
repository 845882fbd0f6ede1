"""Seeded synthetic futon weight packs and token-id batches.

Writes the pack format the reference loads (``native/safetensors.go:6-15``,
``native/manifest.go:20-37``): ``config.json`` (sorted keys),
``model.safetensors`` (F32, tensors sorted by name, compact sorted-key JSON
header padded with spaces to a multiple of 8, as
``scripts/gen-native-embed-fixtures.py:189-207`` writes it), ``vocab.txt``
and ``manifest.json`` (per-member sha256 + size and the exact
``tensor_names`` set).

Randomness is a self-contained splitmix64 stream per tensor, turned into
normals with Box–Muller, so every host regenerates bit-identical packs.

Workloads (embedding-encoder shapes; seeds: ids 42+c, weights 1234+c):

====  ======================  =====================================================
c     name                    shape / batch
====  ======================  =====================================================
0     minilm-l6               6L H384 A12 I1536 GELU abs-pos, mean; B32, L 8..128
1     bge-small               12L H384 A12 I1536 GELU abs-pos, CLS; B256, L 16..128
2     bert-base               12L H768 A12 I3072 GELU abs-pos, mean; B128, L=512
3     nomic-bert              12L H768 A12 SwiGLU I3072 RoPE θ=1000, no biases,
                              mean + Matryoshka 256; B16, L 512..2048
4     bge-small-q8            bge-small with int8 per-row weights (stored
                              dequantized); B1024, L 8..64
====  ======================  =====================================================
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
from dataclasses import dataclass, field

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def _splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 started at seed (wrapping uint64 arithmetic)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniforms(seed: int, n: int) -> np.ndarray:
    """n float64 uniforms in [0, 1) (53-bit)."""
    return (_splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normals(seed: int, n: int) -> np.ndarray:
    """n standard normals (Box–Muller cosine branch over consecutive pairs)."""
    u = uniforms(seed, 2 * n).reshape(n, 2)
    r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
    return r * np.cos(2.0 * np.pi * u[:, 1])


def _stream_seed(seed: int, name: str) -> int:
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return int.from_bytes(h[:8], "little")


def _quantize_dequantize_q8(w: np.ndarray) -> np.ndarray:
    """Per-row absmax int8 then back to float32 (native/quant.go:42-70):
    scale = f32(amax)/127, code = round-half-away(v·127/amax) clamped ±127."""
    amax = np.abs(w).max(axis=1).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(amax > 0, 127.0 / np.where(amax > 0, amax.astype(np.float64), 1.0), 0.0)
    x = w.astype(np.float64) * inv[:, None]
    q = np.clip(np.sign(x) * np.floor(np.abs(x) + 0.5), -127, 127)
    return (q.astype(np.float32) * scale[:, None]).astype(np.float32)


@dataclass
class Workload:
    index: int
    name: str
    config: dict
    batch: int
    len_lo: int
    len_hi: int
    out_dim: int = 0
    q8: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def weight_seed(self) -> int:
        return 1234 + self.index

    @property
    def ids_seed(self) -> int:
        return 42 + self.index


def _bert_cfg(model_id, layers, hidden, heads, inter, pooling):
    return {
        "pack_format": 1, "model_id": model_id,
        "hidden_size": hidden, "num_layers": layers, "num_heads": heads,
        "intermediate_size": inter, "vocab_size": 30522, "type_vocab_size": 2,
        "max_seq_len": 512, "layer_norm_eps": 1e-12,
        "position_encoding": "absolute", "activation": "gelu",
        "pooling": pooling, "normalize": True,
        "tokenizer": {"cls_token": "[CLS]", "do_lower_case": True, "pad_token": "[PAD]",
                      "sep_token": "[SEP]", "tokenize_chinese_chars": True, "unk_token": "[UNK]"},
    }


def workloads() -> list[Workload]:
    nomic = _bert_cfg("nomic-bert-synthetic", 12, 768, 12, 3072, "mean")
    nomic.update({"vocab_size": 30528, "max_seq_len": 2048, "position_encoding": "rope",
                  "rope_theta": 1000.0, "activation": "swiglu",
                  "matryoshka": {"layernorm": True, "dims": [768, 512, 256, 128, 64]}})
    return [
        Workload(0, "minilm-l6", _bert_cfg("minilm-l6-synthetic", 6, 384, 12, 1536, "mean"), 32, 8, 128),
        Workload(1, "bge-small", _bert_cfg("bge-small-synthetic", 12, 384, 12, 1536, "cls"), 256, 16, 128),
        Workload(2, "bert-base", _bert_cfg("bert-base-synthetic", 12, 768, 12, 3072, "mean"), 128, 512, 512),
        Workload(3, "nomic-bert", nomic, 16, 512, 2048, out_dim=256, extra={"biases": False}),
        Workload(4, "bge-small-q8", _bert_cfg("bge-small-q8-synthetic", 12, 384, 12, 1536, "cls"), 1024, 8, 64,
                 q8=True),
    ]


def workload(name: str) -> Workload:
    for w in workloads():
        if w.name == name:
            return w
    raise KeyError(name)


def tensor_specs(cfg: dict, biases: bool = True) -> list[tuple[str, tuple, str]]:
    """(name, shape, kind) for every tensor of a pack; kind ∈ mat|bias|gamma|beta.
    Canonical names follow native/model.go:189-256."""
    h, inter = cfg["hidden_size"], cfg["intermediate_size"]
    out = [("embeddings.word", (cfg["vocab_size"], h), "mat")]
    if cfg["position_encoding"] == "absolute":
        out.append(("embeddings.position", (cfg["max_seq_len"], h), "mat"))
    if cfg.get("type_vocab_size", 0) > 0:
        out.append(("embeddings.token_type", (cfg["type_vocab_size"], h), "mat"))
    out += [("embeddings.norm.weight", (h,), "gamma"), ("embeddings.norm.bias", (h,), "beta")]
    for i in range(cfg["num_layers"]):
        p = f"layers.{i}."
        out.append((p + "attn.qkv.weight", (3 * h, h), "mat"))
        if biases:
            out.append((p + "attn.qkv.bias", (3 * h,), "bias"))
        out.append((p + "attn.out.weight", (h, h), "mat"))
        if biases:
            out.append((p + "attn.out.bias", (h,), "bias"))
        out += [(p + "norm1.weight", (h,), "gamma"), (p + "norm1.bias", (h,), "beta")]
        out.append((p + "mlp.fc1.weight", (inter, h), "mat"))
        if biases:
            out.append((p + "mlp.fc1.bias", (inter,), "bias"))
        if cfg["activation"] == "swiglu":
            out.append((p + "mlp.gate.weight", (inter, h), "mat"))
            if biases:
                out.append((p + "mlp.gate.bias", (inter,), "bias"))
        out.append((p + "mlp.fc2.weight", (h, inter), "mat"))
        if biases:
            out.append((p + "mlp.fc2.bias", (h,), "bias"))
        out += [(p + "norm2.weight", (h,), "gamma"), (p + "norm2.bias", (h,), "beta")]
    return out


def make_tensors(cfg: dict, seed: int, biases: bool = True, q8: bool = False,
                 std: float = 0.02) -> dict[str, np.ndarray]:
    """Seeded weights: matrices/tables and biases N(0, std); LN γ = 1 + N(0, std),
    β = N(0, std).  q8: layer GEMM weights replaced by their per-row int8
    dequantization, so load-time re-quantization reproduces the codes."""
    out = {}
    for name, shape, kind in tensor_specs(cfg, biases):
        n = int(np.prod(shape))
        v = normals(_stream_seed(seed, name), n) * std
        if kind == "gamma":
            v = 1.0 + v
        a = v.astype(np.float32).reshape(shape)
        if q8 and kind == "mat" and name.startswith("layers."):
            a = _quantize_dequantize_q8(a)
        out[name] = a
    return out


def _sha256_file(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def write_safetensors(tensors: dict[str, np.ndarray], path: str, dtype: str = "F32") -> None:
    np_dtype, size = {"F32": ("<f4", 4), "F16": ("<f2", 2)}[dtype]
    names = sorted(tensors)
    header = {}
    offset = 0
    for name in names:
        nbytes = int(np.prod(tensors[name].shape)) * size
        header[name] = {"data_offsets": [offset, offset + nbytes], "dtype": dtype,
                        "shape": list(tensors[name].shape)}
        offset += nbytes
    hjson = json.dumps(header, sort_keys=True, separators=(",", ":")).encode()
    hjson += b" " * ((8 - (8 + len(hjson)) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hjson)))
        f.write(hjson)
        for name in names:
            f.write(np.ascontiguousarray(tensors[name]).astype(np_dtype, copy=False).tobytes())


def default_vocab_path() -> str:
    here = os.path.dirname(os.path.abspath(__file__))
    return os.path.join(os.path.dirname(here), "tests", "golden", "vocab_bert_uncased.txt")


def write_pack(pack_dir: str, cfg: dict, tensors: dict[str, np.ndarray], vocab_path: str | None = None,
               dtype: str = "F32") -> str:
    """Writes a complete futon pack (config, weights, vocab, manifest)."""
    os.makedirs(pack_dir, exist_ok=True)
    with open(os.path.join(pack_dir, "config.json"), "w", encoding="utf-8", newline="\n") as f:
        f.write(json.dumps(cfg, indent=2, sort_keys=True) + "\n")
    write_safetensors(tensors, os.path.join(pack_dir, "model.safetensors"), dtype)
    with open(vocab_path or default_vocab_path(), "rb") as src:
        vocab = src.read()
    with open(os.path.join(pack_dir, "vocab.txt"), "wb") as f:
        f.write(vocab)
    members = {}
    for m in ("config.json", "model.safetensors", "vocab.txt"):
        p = os.path.join(pack_dir, m)
        members[m] = {"sha256": _sha256_file(p), "size": os.path.getsize(p)}
    manifest = {"pack_format": 1, "model_id": cfg["model_id"], "created_by": "futon_amd.synth",
                "members": members, "tensor_names": sorted(tensors)}
    with open(os.path.join(pack_dir, "manifest.json"), "w", encoding="utf-8", newline="\n") as f:
        f.write(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    return pack_dir


def ensure_workload_pack(w: Workload, root: str) -> str:
    """Writes w's pack under root/<name> unless an identical one exists."""
    d = os.path.join(root, w.name)
    stamp = os.path.join(d, ".synth-stamp")
    key = json.dumps({"cfg": w.config, "seed": w.weight_seed, "q8": w.q8, "extra": w.extra}, sort_keys=True)
    if os.path.exists(stamp) and open(stamp).read() == key:
        return d
    t = make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    write_pack(d, w.config, t)
    with open(stamp, "w") as f:
        f.write(key)
    return d


# ── token ids ────────────────────────────────────────────────────────────────
_ZIPF_CDF = None


def _zipf_cdf() -> np.ndarray:
    global _ZIPF_CDF
    if _ZIPF_CDF is None:
        ranks = np.arange(1, 29523, dtype=np.float64)
        w = ranks ** -1.1
        _ZIPF_CDF = np.cumsum(w) / w.sum()
    return _ZIPF_CDF


def make_batch(seed: int, batch: int, len_lo: int, len_hi: int):
    """[CLS]=101 + Zipf(s=1.1) ids over ranks 1..29522 → ids 1000..30521 +
    [SEP]=102; lengths uniform in [len_lo, len_hi] (total, with CLS/SEP).
    Returns (ids int32 [T], offsets int32 [batch+1]) — packed, unpadded."""
    u_len = uniforms(seed, batch)
    lens = (len_lo + np.floor(u_len * (len_hi - len_lo + 1))).astype(np.int64)
    lens = np.minimum(lens, len_hi)
    offsets = np.zeros(batch + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(lens)
    total = int(offsets[-1])
    u_id = uniforms(seed ^ 0x5EED5EED5EED5EED, total)
    rank = np.searchsorted(_zipf_cdf(), u_id, side="right") + 1
    rank = np.minimum(rank, 29522)
    ids = (999 + rank).astype(np.int32)
    ids[offsets[:-1]] = 101
    ids[offsets[1:] - 1] = 102
    return ids, offsets.astype(np.int32)
