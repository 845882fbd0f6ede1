"""Host side of the futon encoder on MI355X, mirroring the reference's
``native`` package API for the forward path:

* ``LoadModel(dir, threads)``          — native/model.go:112-132
* ``Model.Config()``                   — native/model.go:298
* ``Model.EncodeTokens(ids, out_dim)`` — native/model.go:335-457
* ``Model.EncodeBatch(batch, out_dim)``— one device call for many sequences,
                                          what Provider.EmbedBatch drives
                                          (native/provider.go:152-202)
* ``PackConfig`` + ``LoadPackConfig``  — native/config.go:54-187
* ``LoadSafetensors(Raw)``             — native/safetensors.go:79-221
* manifest verification               — native/manifest.go:46-104

Every validation happens here, on the host, before the C ABI is called —
the same split the reference's Go host keeps in front of its kernels.  The
forward itself runs only in libfuton_hip.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import math
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
MAX_HEADER_BYTES = 16 << 20
MANIFEST_MEMBERS = ("config.json", "model.safetensors", "vocab.txt")


class PackError(ValueError):
    """A pack failed validation (the reference's load-time errors)."""


# ── config (native/config.go) ────────────────────────────────────────────────
@dataclass
class MatryoshkaConfig:
    layernorm: bool = False
    dims: list = field(default_factory=list)


@dataclass
class PackConfig:
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

    def Validate(self) -> None:  # native/config.go:119-171
        mid = self.model_id
        if self.pack_format != PACK_FORMAT_VERSION:
            raise PackError(f"pack: unsupported pack_format {self.pack_format} (loader supports {PACK_FORMAT_VERSION})")
        if not mid:
            raise PackError("pack: model_id missing")
        if self.hidden_size <= 0 or self.num_layers <= 0 or self.num_heads <= 0 or self.intermediate_size <= 0:
            raise PackError(f"pack {mid}: non-positive architecture dimension")
        if self.hidden_size % self.num_heads:
            raise PackError(f"pack {mid}: hidden_size {self.hidden_size} not divisible by num_heads {self.num_heads}")
        if self.vocab_size <= 0 or self.max_seq_len <= 2:
            raise PackError(f"pack {mid}: invalid vocab_size/max_seq_len")
        if self.max_trained_positions < 0 or 0 < self.max_trained_positions <= 2:
            raise PackError(f"pack {mid}: invalid max_trained_positions {self.max_trained_positions}")
        if self.layer_norm_eps <= 0:
            raise PackError(f"pack {mid}: layer_norm_eps must be positive")
        if self.position_encoding == POS_ROPE:
            if self.rope_theta <= 0:
                raise PackError(f"pack {mid}: rope position encoding requires rope_theta > 0")
        elif self.position_encoding != POS_ABSOLUTE:
            raise PackError(f"pack {mid}: unknown position_encoding {self.position_encoding!r}")
        if self.activation not in (ACT_GELU, ACT_SWIGLU):
            raise PackError(f"pack {mid}: unknown activation {self.activation!r}")
        if self.pooling not in (POOL_MEAN, POOL_CLS):
            raise PackError(f"pack {mid}: unknown pooling {self.pooling!r}")
        if self.pre_norm:
            raise PackError(f"pack {mid}: pre_norm is declared but not yet implemented — refusing to run the "
                            "wrong architecture")
        if self.matryoshka is not None:
            for d in self.matryoshka.dims:
                if d <= 0 or d > self.hidden_size:
                    raise PackError(f"pack {mid}: matryoshka dim {d} outside (0,{self.hidden_size}]")


def LoadPackConfig(dir: str) -> PackConfig:  # native/config.go:174-187
    try:
        raw = open(os.path.join(dir, "config.json"), "rb").read()
    except OSError as e:
        raise PackError(f"pack: read config: {e}") from e
    try:
        d = json.loads(raw)
    except ValueError as e:
        raise PackError(f"pack: parse config: {e}") from e
    cfg = PackConfig.from_dict(d)
    cfg.Validate()
    return cfg


# ── safetensors (native/safetensors.go) ──────────────────────────────────────
def ParseSafetensors(raw: bytes, keep_f16: bool = False) -> dict:
    """Strict parse: shapes × dtype must match each span, spans must tile the
    data section exactly (no gap, overlap or trailing bytes)."""
    if len(raw) < 8:
        raise PackError(f"safetensors: file too small ({len(raw)} bytes) for header length prefix")
    (hl,) = struct.unpack("<Q", raw[:8])
    if hl > MAX_HEADER_BYTES:
        raise PackError(f"safetensors: header length {hl} exceeds limit {MAX_HEADER_BYTES}")
    if len(raw) < 8 + hl:
        raise PackError(f"safetensors: declared header length {hl} exceeds file size {len(raw)}")
    try:
        header = json.loads(raw[8:8 + hl])
    except ValueError as e:
        raise PackError(f"safetensors: parse header JSON: {e}") from e
    if not isinstance(header, dict):
        raise PackError("safetensors: header is not an object")
    data = memoryview(raw)[8 + hl:]
    tensors, spans = {}, []
    for name, e in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(e, dict):
            raise PackError(f"safetensors: tensor {name!r}: parse entry: not an object")
        dt = e.get("dtype")
        if dt == "F32":
            esz, npdt = 4, "<f4"
        elif dt == "F16":
            esz, npdt = 2, "<f2"
        else:
            raise PackError(f"safetensors: tensor {name!r}: unsupported dtype {dt!r} (want F32 or F16)")
        shape = e.get("shape")
        offs = e.get("data_offsets")
        if not isinstance(shape, list) or not all(isinstance(d, int) for d in shape):
            raise PackError(f"safetensors: tensor {name!r}: parse entry: bad shape")
        if not isinstance(offs, list) or len(offs) != 2 or not all(isinstance(o, int) for o in offs):
            raise PackError(f"safetensors: tensor {name!r}: parse entry: bad data_offsets")
        n = 1
        for d in shape:
            if d < 0:
                raise PackError(f"safetensors: tensor {name!r}: negative dimension {d}")
            n *= d
            if n >= 1 << 64:
                raise PackError(f"safetensors: tensor {name!r}: shape {shape} element count overflows")
        if n > (2 ** 63 - 1) // esz:
            raise PackError(f"safetensors: tensor {name!r}: shape {shape} byte size overflows")
        b, en = offs
        if b < 0 or en < b or en > len(data):
            raise PackError(f"safetensors: tensor {name!r}: offsets [{b},{en}) outside data section of "
                            f"{len(data)} bytes")
        if en - b != n * esz:
            raise PackError(f"safetensors: tensor {name!r}: shape {shape} × {dt} needs {n * esz} bytes, "
                            f"offsets span {en - b}")
        arr = np.frombuffer(data[b:en], dtype=npdt).reshape(shape)
        if dt == "F16" and not keep_f16:
            arr = arr.astype(np.float32)
        tensors[name] = arr
        spans.append((b, en, name))
    spans.sort()
    cursor = 0
    for b, en, name in spans:
        if b != cursor:
            raise PackError(f"safetensors: tensor {name!r} begins at {b}, expected {cursor} (overlap or gap)")
        cursor = en
    if cursor != len(data):
        raise PackError(f"safetensors: data section is {len(data)} bytes but tensors cover {cursor}")
    return tensors


def LoadSafetensors(path: str) -> dict:
    return ParseSafetensors(open(path, "rb").read())


def LoadSafetensorsRaw(path: str) -> dict:
    return ParseSafetensors(open(path, "rb").read(), keep_f16=True)


# ── manifest (native/manifest.go) ────────────────────────────────────────────
def sha256_file(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def load_and_verify_manifest(dir: str) -> dict:
    try:
        raw = open(os.path.join(dir, "manifest.json"), "rb").read()
    except OSError as e:
        raise PackError(f"pack {dir}: manifest.json unreadable (refusing to load an unverifiable pack): {e}") from e
    try:
        man = json.loads(raw)
    except ValueError as e:
        raise PackError(f"pack {dir}: manifest.json malformed: {e}") from e
    members = man.get("members") or {}
    for member in MANIFEST_MEMBERS:
        meta = members.get(member)
        if meta is None:
            raise PackError(f"pack {dir}: manifest records no entry for {member}")
        path = os.path.join(dir, member)
        try:
            size = os.path.getsize(path)
        except OSError as e:
            raise PackError(f"pack {dir}: member {member}: {e}") from e
        if size != meta.get("size"):
            raise PackError(f"pack {dir}: member {member} is {size} bytes, manifest records {meta.get('size')}")
        got = sha256_file(path)
        if got != meta.get("sha256"):
            raise PackError(f"pack {dir}: member {member} sha256 {got} does not match manifest {meta.get('sha256')} "
                            "(tampered or corrupt — rebuild the pack)")
    return man


def verify_tensor_names(man: dict, tensors: dict) -> None:
    want = man.get("tensor_names")
    if want is None:
        return
    got = sorted(tensors)
    want = sorted(want)
    mid = man.get("model_id", "")
    if len(got) != len(want):
        raise PackError(f"pack {mid}: {len(got)} tensors on disk, manifest records {len(want)} — tensor set drifted")
    for g, w in zip(got, want):
        if g != w:
            raise PackError(f"pack {mid}: tensor set drifted from manifest (first difference: {g!r} vs recorded {w!r})")


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
    """native/model.go:112-132: verify the manifest, load and validate the
    config, parse the weights strictly, check the recorded tensor-name set,
    then upload (newModel's shape checks run at the C ABI).  ``threads`` is
    accepted for API parity; the device decides its own parallelism."""
    man = load_and_verify_manifest(dir)
    cfg = LoadPackConfig(dir)
    if man.get("model_id") != cfg.model_id:
        raise PackError(f"pack {cfg.model_id}: manifest is for {man.get('model_id')!r} — mixed pack contents")
    try:
        tensors = LoadSafetensorsRaw(os.path.join(dir, "model.safetensors"))
    except PackError as e:
        raise PackError(f"pack {cfg.model_id}: {e}") from e
    except OSError as e:
        raise PackError(f"safetensors: read {dir}: {e}") from e
    verify_tensor_names(man, tensors)
    return Model(cfg, tensors, device=device, q8=q8)
