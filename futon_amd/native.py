"""Python binding of the host side of the futon encoder on MI355X.

The host side itself is C++ (include/futon_native.hpp, futon_amd/csrc/host):
pack loading with the reference's validation, the WordPiece tokenizer and
the Provider.  This module exposes it through the C ABI (include/futon_host.h
and include/futon_hip.h) under the reference's names, so tests read like the
reference's own:

* ``LoadPackConfig`` / ``PackConfig``  — native/config.go:54-187
* ``ParseSafetensors`` / ``LoadSafetensors(Raw)`` — native/safetensors.go:79-221
* ``LoadPack``                         — the host half of LoadModel, model.go:112-131
* ``LoadModel(dir, threads)``          — native/model.go:112-132
* ``Model.EncodeTokens`` / ``EncodeBatch`` — native/model.go:335-457
* ``Tokenizer`` / ``NewTokenizer``     — native/tokenizer.go:94-176
* ``New`` / ``Provider``               — native/provider.go:70-290
* ``futon_New``                        — futon.go:84-98

The forward runs only in libfuton_hip.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import os
import struct
import threading
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import FutonError

PACK_FORMAT_VERSION = 1
POS_ABSOLUTE, POS_ROPE = "absolute", "rope"
ACT_GELU, ACT_SWIGLU = "gelu", "swiglu"
POOL_MEAN, POOL_CLS = "mean", "cls"
ENV_NATIVE_Q8 = "FUTON_NATIVE_Q8"


class PackError(ValueError):
    """A pack failed validation (the reference's load-time errors)."""


def _raise(rc: int, what: str) -> None:
    if rc == _lib.FH_OK:
        return
    msg = _lib.last_error()
    if rc == _lib.FH_EINVAL:
        raise PackError(msg)
    raise FutonError(rc, f"{what}: {msg}")


# ── config (native/config.go) ────────────────────────────────────────────────
@dataclass
class MatryoshkaConfig:
    layernorm: bool = False
    dims: list = field(default_factory=list)


@dataclass
class PackConfig:
    """Field view of a pack's config.json.  Validation is the C++ host
    layer's (PackConfig::Validate); this object only carries the values."""
    pack_format: int = 0
    model_id: str = ""
    hidden_size: int = 0
    num_layers: int = 0
    num_heads: int = 0
    intermediate_size: int = 0
    vocab_size: int = 0
    type_vocab_size: int = 0
    max_seq_len: int = 0
    layer_norm_eps: float = 0.0
    position_encoding: str = ""
    rope_theta: float = 0.0
    max_trained_positions: int = 0
    activation: str = ""
    pre_norm: bool = False
    pooling: str = ""
    normalize: bool = False
    matryoshka: Optional[MatryoshkaConfig] = None
    tokenizer: dict = field(default_factory=dict)
    prefixes: dict = field(default_factory=dict)

    @classmethod
    def from_dict(cls, d: dict) -> "PackConfig":
        c = cls()
        for k, v in d.items():
            if k == "matryoshka":
                c.matryoshka = None if v is None else MatryoshkaConfig(bool(v.get("layernorm", False)),
                                                                       list(v.get("dims") or []))
            elif hasattr(c, k):
                setattr(c, k, v)
        return c

    def EffectiveMaxSeqLen(self) -> int:  # native/config.go:111-116
        if 0 < self.max_trained_positions < self.max_seq_len:
            return self.max_trained_positions
        return self.max_seq_len


def LoadPackConfig(dir: str) -> PackConfig:
    """native/config.go:174-187 — read and validate (in C++) <dir>/config.json."""
    L = _lib.load()
    c = _lib.FhConfig()
    eff = ctypes.c_int32()
    _raise(L.fh_pack_config_load(dir.encode(), ctypes.byref(c), ctypes.byref(eff)), "LoadPackConfig")
    with open(os.path.join(dir, "config.json"), "rb") as f:
        return PackConfig.from_dict(json.loads(f.read()))


# ── safetensors (native/safetensors.go) ──────────────────────────────────────
def ParseSafetensors(raw: bytes, keep_f16: bool = False) -> dict:
    """Strict parse of a safetensors image: the C++ reader validates it
    (shapes × dtype match each span, spans tile the data section exactly),
    then the tensors are viewed as numpy arrays."""
    n = ctypes.c_int32()
    _raise(_lib.load().fh_safetensors_check(raw, len(raw), ctypes.byref(n)), "ParseSafetensors")
    (hl,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + hl])
    data = memoryview(raw)[8 + hl:]
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        b, en = e["data_offsets"][:2]
        arr = np.frombuffer(data[b:en], dtype="<f4" if e["dtype"] == "F32" else "<f2").reshape(e["shape"])
        out[name] = arr.astype(np.float32) if (e["dtype"] == "F16" and not keep_f16) else arr
    return out


def LoadSafetensors(path: str) -> dict:
    with open(path, "rb") as f:
        return ParseSafetensors(f.read())


def LoadSafetensorsRaw(path: str) -> dict:
    with open(path, "rb") as f:
        return ParseSafetensors(f.read(), keep_f16=True)


def sha256_file(path: str) -> str:
    """Hex SHA-256 of a file (test helper for re-hashing manifests)."""
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


class Pack:
    """native/model.go:112-131 up to the device: manifest verification,
    config, model_id agreement, safetensors, tensor-name set — all in C++."""

    def __init__(self, dir: str):
        self._h = None
        h = ctypes.c_void_p()
        _raise(_lib.load().fh_pack_load(dir.encode(), ctypes.byref(h)), "LoadPack")
        self._h = h.value
        self.dir = dir
        with open(os.path.join(dir, "config.json"), "rb") as f:
            self.config = PackConfig.from_dict(json.loads(f.read()))

    @property
    def model_id(self) -> str:
        buf = ctypes.create_string_buffer(512)
        _lib.load().fh_pack_model_id(self._h, buf, 512)
        return buf.value.decode()

    def tensor_count(self) -> int:
        return _lib.load().fh_pack_tensor_count(self._h)

    def close(self) -> None:
        if self._h is not None:
            _lib.load().fh_pack_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def LoadPack(dir: str) -> Pack:
    return Pack(dir)


# ── model ────────────────────────────────────────────────────────────────────
def _fh_config(cfg: PackConfig, q8: bool) -> _lib.FhConfig:
    c = _lib.FhConfig()
    c.hidden_size, c.num_layers, c.num_heads = cfg.hidden_size, cfg.num_layers, cfg.num_heads
    c.intermediate_size, c.vocab_size = cfg.intermediate_size, cfg.vocab_size
    c.type_vocab_size, c.max_seq_len = cfg.type_vocab_size, cfg.max_seq_len
    c.max_trained_positions = cfg.max_trained_positions
    c.layer_norm_eps = cfg.layer_norm_eps
    c.position_encoding = _lib.FH_POS_ROPE if cfg.position_encoding == POS_ROPE else _lib.FH_POS_ABSOLUTE
    c.rope_theta = cfg.rope_theta or 0.0
    c.activation = _lib.FH_ACT_SWIGLU if cfg.activation == ACT_SWIGLU else _lib.FH_ACT_GELU
    c.pooling = _lib.FH_POOL_CLS if cfg.pooling == POOL_CLS else _lib.FH_POOL_MEAN
    c.normalize = int(bool(cfg.normalize))
    c.matryoshka = int(cfg.matryoshka is not None)
    c.matryoshka_layernorm = int(bool(cfg.matryoshka and cfg.matryoshka.layernorm))
    c.q8 = int(bool(q8))
    return c


class Model:
    """A pack resident on one MI355X.  Safe for concurrent use (the device
    call is serialized per model)."""

    def __init__(self, cfg: PackConfig, tensors: dict, device: int = 0, q8: Optional[bool] = None):
        self._h = None
        L = _lib.load()
        if q8 is None:
            q8 = os.environ.get(ENV_NATIVE_Q8) == "1"
        self.cfg = cfg
        self.q8 = bool(q8)
        names = list(tensors)
        arr = (_lib.FhTensor * max(1, len(names)))()
        keep = []
        for i, n in enumerate(names):
            a = tensors[n]
            if a.dtype == np.float16 or a.dtype == np.dtype("<f2"):
                a = np.ascontiguousarray(a, dtype="<f2")
                dt = _lib.FH_DTYPE_F16
            else:
                a = np.ascontiguousarray(a, dtype=np.float32)
                dt = _lib.FH_DTYPE_F32
            if a.ndim > 4:
                raise PackError(f"tensor {n!r} has rank {a.ndim} > 4")
            keep.append(a)
            bname = n.encode()
            keep.append(bname)
            arr[i].name = bname
            arr[i].dtype = dt
            arr[i].rank = a.ndim
            for j, d in enumerate(a.shape):
                arr[i].shape[j] = d
            arr[i].data = a.ctypes.data
        h = ctypes.c_void_p()
        rc = L.fh_model_create(ctypes.byref(_fh_config(cfg, self.q8)), arr, len(names), device, ctypes.byref(h))
        if rc != _lib.FH_OK:
            msg = _lib.last_error()
            if rc == _lib.FH_EINVAL:
                raise PackError(msg)
            _lib.check(rc, "fh_model_create")
        self._h = h.value
        self._lock = threading.Lock()

    @classmethod
    def _adopt(cls, cfg: PackConfig, handle: int, q8: bool) -> "Model":
        m = cls.__new__(cls)
        m._h = handle
        m.cfg = cfg
        m.q8 = q8
        m._lock = threading.Lock()
        return m

    @property
    def handle(self) -> int:
        if self._h is None:
            raise FutonError(_lib.FH_EINVAL, "native: model is closed")
        return self._h

    def Config(self) -> PackConfig:
        return self.cfg

    def close(self) -> None:
        if self._h is not None:
            _lib.load().fh_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_bytes(self) -> int:
        return _lib.load().fh_model_device_bytes(self.handle)

    def EncodeTokens(self, ids: Sequence[int], out_dim: int = 0, cancel=None) -> np.ndarray:
        """One sequence (already [CLS] … [SEP]) → pooled vector."""
        return self.EncodeBatch([ids], out_dim, cancel)[0]

    def EncodeBatch(self, batch: Sequence[Sequence[int]], out_dim: int = 0, cancel=None) -> np.ndarray:
        lens = [len(s) for s in batch]
        offsets = np.zeros(len(batch) + 1, dtype=np.int32)
        offsets[1:] = np.cumsum(lens, dtype=np.int64)
        ids = np.concatenate([np.asarray(s, dtype=np.int64) for s in batch]) if batch else np.zeros(0, np.int64)
        if ids.size and (ids.min() < -2 ** 31 or ids.max() >= 2 ** 31):
            raise FutonError(_lib.FH_EINVAL, "native: token id outside int32")
        return self.EncodePacked(ids.astype(np.int32), offsets, out_dim, cancel)

    def EncodePacked(self, ids: np.ndarray, offsets: np.ndarray, out_dim: int = 0, cancel=None) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        offsets = np.ascontiguousarray(offsets, dtype=np.int32)
        nseq = offsets.size - 1
        od = self.cfg.hidden_size if out_dim == 0 else out_dim
        out = np.zeros((max(nseq, 0), max(od, 0)), dtype=np.float32)
        if nseq <= 0:
            return out
        cflag = None
        if cancel is not None:
            cflag = cancel if isinstance(cancel, ctypes.c_int32) else ctypes.c_int32(int(bool(cancel)))
        rc = _lib.load().fh_encode(self.handle, ids.ctypes.data, offsets.ctypes.data, nseq, out_dim,
                                   out.ctypes.data, ctypes.addressof(cflag) if cflag is not None else None)
        _lib.check(rc, "fh_encode")
        return out

    def EncodeDevice(self, d_ids: int, d_offsets: int, nseq: int, total: int, max_len: int, out_dim: int,
                     d_out: int, stream: int = 0, h_offsets: Optional[np.ndarray] = None) -> None:
        hp = None
        if h_offsets is not None:
            h_offsets = np.ascontiguousarray(h_offsets, dtype=np.int32)
            hp = h_offsets.ctypes.data
        rc = _lib.load().fh_encode_device(self.handle, d_ids, d_offsets, nseq, total, max_len, out_dim, d_out,
                                          stream or None, hp)
        _lib.check(rc, "fh_encode_device")

    # profiling / test hooks
    def profile_enable(self, on: bool = True) -> None:
        _lib.check(_lib.load().fh_profile_enable(self.handle, int(on)))

    def profile_reset(self) -> None:
        _lib.check(_lib.load().fh_profile_reset(self.handle))

    def profile_read(self) -> dict:
        n = 32
        names = (ctypes.c_char_p * n)()
        ms = (ctypes.c_double * n)()
        launches = (ctypes.c_int64 * n)()
        flops = (ctypes.c_double * n)()
        byts = (ctypes.c_double * n)()
        k = _lib.load().fh_profile_read(self.handle, names, ms, launches, flops, byts, n)
        if k < 0:
            _lib.check(k)
        return {names[i].decode(): {"ms": ms[i], "launches": launches[i], "flops": flops[i], "bytes": byts[i]}
                for i in range(min(k, n))}

    def debug_cancel_after(self, n: int) -> None:
        _lib.check(_lib.load().fh_debug_cancel_after(self.handle, n))

    def checkpoints_per_call(self) -> int:
        return _lib.load().fh_checkpoints_per_call(self.handle)


def LoadModel(dir: str, threads: int = 0, device: int = 0, q8: Optional[bool] = None) -> Model:
    """native/model.go:112-132: the C++ host layer verifies the manifest,
    loads and validates the config, parses the weights strictly and checks
    the recorded tensor-name set (LoadPack); newModel's shape checks and the
    upload run at the C ABI.  ``threads`` is accepted for API parity."""
    if q8 is None:
        q8 = os.environ.get(ENV_NATIVE_Q8) == "1"
    pack = LoadPack(dir)
    try:
        h = ctypes.c_void_p()
        _raise(_lib.load().fh_pack_create_model(pack._h, int(bool(q8)), device, ctypes.byref(h)), "LoadModel")
        return Model._adopt(pack.config, h.value, bool(q8))
    finally:
        pack.close()


# ── tokenizer (native/tokenizer.go) ──────────────────────────────────────────
class Tokenizer:
    """native.NewTokenizer / Tokenizer.Encode (native/tokenizer.go:94-176),
    implemented in C++."""

    def __init__(self, vocab_path: str, cfg: Optional[dict] = None):
        cfg = cfg or {}
        c = _lib.FhTokenizerConfig()
        c.do_lower_case = int(bool(cfg.get("do_lower_case", False)))
        c.tokenize_chinese_chars = int(bool(cfg.get("tokenize_chinese_chars", False)))
        c.max_input_chars_per_word = int(cfg.get("max_input_chars_per_word", 0) or 0)
        self._keep = []
        for k in ("cls_token", "sep_token", "unk_token", "pad_token", "mask_token"):
            v = cfg.get(k)
            if v:
                b = v.encode()
                self._keep.append(b)
                setattr(c, k, b)
        self._h = None
        h = ctypes.c_void_p()
        _raise(_lib.load().fh_tokenizer_new(vocab_path.encode(), ctypes.byref(c), ctypes.byref(h)), "NewTokenizer")
        self._h = h.value

    def Encode(self, text, max_seq_len: int) -> list:
        raw = text.encode("utf-8", "surrogatepass") if isinstance(text, str) else bytes(text)
        L = _lib.load()
        n = ctypes.c_int32()
        cap = max(2, min(max_seq_len, 1 << 20))
        buf = (ctypes.c_int32 * cap)()
        _raise(L.fh_tokenizer_encode(self._h, raw, len(raw), max_seq_len, buf, cap, ctypes.byref(n)), "Encode")
        if n.value > cap:
            buf = (ctypes.c_int32 * n.value)()
            _raise(L.fh_tokenizer_encode(self._h, raw, len(raw), max_seq_len, buf, n.value, ctypes.byref(n)), "Encode")
        return list(buf[:n.value])

    def VocabSize(self) -> int:
        return _lib.load().fh_tokenizer_vocab_size(self._h)

    def close(self) -> None:
        if self._h is not None:
            _lib.load().fh_tokenizer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def NewTokenizer(vocab_path: str, cfg: Optional[dict] = None) -> Tokenizer:
    return Tokenizer(vocab_path, cfg)


# ── provider (native/provider.go) ─────────────────────────────────────────────
class Provider:
    """native.New / Provider (native/provider.go:70-290) over the C++
    host layer: host tokenization, one packed device call per batch chunk."""

    def __init__(self, handle: int):
        self._h = handle

    def _handle(self) -> int:
        if self._h is None:
            raise FutonError(_lib.FH_EINVAL, "native: provider is freed")
        return self._h

    def Dimensions(self) -> int:
        return _lib.load().fh_provider_dimensions(self._handle())

    def ModelName(self) -> str:
        buf = ctypes.create_string_buffer(512)
        _lib.load().fh_provider_model_name(self._handle(), buf, 512)
        return buf.value.decode()

    def IsAvailable(self) -> bool:
        return bool(_lib.load().fh_provider_is_available(self._handle()))

    def Embed(self, text, cancel=None) -> np.ndarray:
        return self.EmbedBatch([text], cancel)[0]

    def EmbedBatch(self, texts: Sequence, cancel=None) -> np.ndarray:
        n = len(texts)
        dim = self.Dimensions()
        out = np.zeros((n, dim), dtype=np.float32)
        if n == 0:
            return out
        raws = [t.encode("utf-8", "surrogatepass") if isinstance(t, str) else bytes(t) for t in texts]
        ptrs = (ctypes.c_char_p * n)(*raws)
        lens = (ctypes.c_size_t * n)(*[len(r) for r in raws])
        cflag = None
        if cancel is not None:
            cflag = cancel if isinstance(cancel, ctypes.c_int32) else ctypes.c_int32(int(bool(cancel)))
        rc = _lib.load().fh_provider_embed_batch(self._handle(), ptrs, lens, n, out.ctypes.data,
                                                 ctypes.addressof(cflag) if cflag is not None else None)
        if rc != _lib.FH_OK:
            raise FutonError(rc, _lib.last_error())
        return out

    def Close(self) -> None:
        if self._h is not None:
            _lib.load().fh_provider_close(self._h)

    def free(self) -> None:
        if self._h is not None:
            _lib.load().fh_provider_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def New(pack_dir: str, dimensions: int = 0, threads: int = 0) -> Provider:
    """native.New(Options{PackDir, Dimensions, Threads})."""
    h = ctypes.c_void_p()
    _raise(_lib.load().fh_provider_new(pack_dir.encode() if pack_dir is not None else None, dimensions, threads,
                                       ctypes.byref(h)), "native.New")
    return Provider(h.value)


def futon_New(model: str = "", models_dir: str = "", model_path: str = "", dimensions: int = 0,
              threads: int = 0) -> Provider:
    """futon.New(Options{Model, ModelsDir, ModelPath, Dimensions, Threads}) for local packs."""
    h = ctypes.c_void_p()
    _raise(_lib.load().fh_futon_new(model.encode(), models_dir.encode(), model_path.encode(), dimensions, threads,
                                    ctypes.byref(h)), "futon.New")
    return Provider(h.value)
