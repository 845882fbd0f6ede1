"""CPU oracle for the futon encoder forward pass — TEST INFRASTRUCTURE ONLY.

ctypes binding of ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this module, and only to compare
against; nothing under ``futon_amd/`` may import it.

Parity status of each function (how it is pinned; see ``tests/test_oracle.py``):

* ``exp_f32``/``gelu_f32``/``sigmoid_f32`` — error bounds against float64 libm
  (the reference's ``native/mathf32_test.go:10-58``) plus exact special values.
* ``f16_to_f32``/``f32_to_f16`` — the reference's known-answer table and
  round-to-nearest-even cases (``native/safetensors_test.go:154-207``) and an
  exhaustive round trip against numpy's IEEE binary16.
* ``quantize_row_q8``/``matmul_t_q8`` — quantizer invariants and the exact
  int64 closed form (``native/quant_test.go:14-100``).
* ``matmul_t`` — float64 naive reference at 1e-4 (``native/kernel_test.go``).
* ``Model.encode`` — the reference's upstream-generated toy goldens
  (``native/testdata/toy/expected.json``) at cosine ≥ 0.99999 / abs ≤ 2e-4
  for both architectures and Matryoshka, and at real shapes against an
  independent torch float64 BERT forward (``tests/golden/``).
"""
from __future__ import annotations

import ctypes
import os
from typing import Mapping

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# FUTON_ORACLE_LIB selects another build of oracle.c (the sanitizer test's).
_LIB_PATH = os.environ.get("FUTON_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    """Compiles liboracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        L.fo_exp_f32.restype = ctypes.c_float
        L.fo_exp_f32.argtypes = [ctypes.c_float]
        L.fo_erfc_pos.restype = ctypes.c_float
        L.fo_erfc_pos.argtypes = [ctypes.c_float]
        L.fo_gelu_f32.restype = ctypes.c_float
        L.fo_gelu_f32.argtypes = [ctypes.c_float]
        L.fo_sigmoid_f32.restype = ctypes.c_float
        L.fo_sigmoid_f32.argtypes = [ctypes.c_float]
        L.fo_f16_to_f32.restype = ctypes.c_float
        L.fo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.fo_f32_to_f16.restype = ctypes.c_uint16
        L.fo_f32_to_f16.argtypes = [ctypes.c_float]
        L.fo_quantize_row_q8.restype = ctypes.c_float
        L.fo_quantize_row_q8.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        for name in ("fo_matmul_t", "fo_matmul_t_f16"):
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3 + [ctypes.c_void_p]
        L.fo_matmul_t_q8.restype = None
        L.fo_matmul_t_q8.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3 + [ctypes.c_void_p]
        L.fo_softmax_scaled.restype = None
        L.fo_softmax_scaled.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_float]
        L.fo_layer_norm_rows.restype = None
        L.fo_layer_norm_rows.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float]
        L.fo_model_create.restype = ctypes.c_void_p
        L.fo_model_create.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int]
        L.fo_model_destroy.restype = None
        L.fo_model_destroy.argtypes = [ctypes.c_void_p]
        L.fo_encode.restype = ctypes.c_int
        L.fo_encode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int]
        L.fo_encode_batch.restype = ctypes.c_int
        L.fo_encode_batch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p,
                                      ctypes.c_int]
        del f32p
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def exp_f32(x: float) -> float:
    return lib().fo_exp_f32(float(x))


def erfc_pos(x: float) -> float:
    return lib().fo_erfc_pos(float(x))


def gelu_f32(x: float) -> float:
    return lib().fo_gelu_f32(float(x))


def sigmoid_f32(x: float) -> float:
    return lib().fo_sigmoid_f32(float(x))


def f16_to_f32(bits: int) -> float:
    return lib().fo_f16_to_f32(int(bits))


def f32_to_f16(x: float) -> int:
    return lib().fo_f32_to_f16(float(x))


def quantize_row_q8(src: np.ndarray):
    src = np.ascontiguousarray(src, dtype=np.float32)
    dst = np.zeros(src.shape, dtype=np.int8)
    scale = lib().fo_quantize_row_q8(_ptr(dst), _ptr(src), src.size)
    return dst, np.float32(scale)


def quantize_q8(w: np.ndarray):
    """Per-row quantization of an n×k matrix (native/quant.go:75-86)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    q = np.zeros(w.shape, dtype=np.int8)
    s = np.zeros(w.shape[0], dtype=np.float32)
    for j in range(w.shape[0]):
        q[j], s[j] = quantize_row_q8(w[j])
    return q, s


def matmul_t(a: np.ndarray, b: np.ndarray, bias=None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    bp = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        bp = _ptr(bias)
    lib().fo_matmul_t(_ptr(out), _ptr(a), _ptr(b), m, n, k, bp)
    return out


def matmul_t_q8(a: np.ndarray, qb: np.ndarray, scales: np.ndarray, bias=None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    qb = np.ascontiguousarray(qb, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    m, k = a.shape
    n = qb.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    bp = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        bp = _ptr(bias)
    lib().fo_matmul_t_q8(_ptr(out), _ptr(a), _ptr(qb), _ptr(scales), m, n, k, bp)
    return out


def softmax_scaled(row: np.ndarray, scale: float) -> np.ndarray:
    r = np.array(row, dtype=np.float32)
    lib().fo_softmax_scaled(_ptr(r), r.size, scale)
    return r


def layer_norm_rows(x: np.ndarray, weight=None, bias=None, eps: float = 1e-12) -> np.ndarray:
    x = np.array(x, dtype=np.float32, ndmin=2)
    rows, h = x.shape
    wp = bp = None
    if weight is not None:
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        wp, bp = _ptr(weight), _ptr(bias)
    lib().fo_layer_norm_rows(_ptr(x), rows, h, wp, bp, eps)
    return x


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("hidden", "layers", "heads", "inter", "vocab", "type_vocab", "max_seq_len", "max_trained")] + [
        ("eps", ctypes.c_double), ("rope", ctypes.c_int), ("rope_theta", ctypes.c_double),
        ("swiglu", ctypes.c_int), ("pool_cls", ctypes.c_int), ("normalize", ctypes.c_int),
        ("matryoshka", ctypes.c_int), ("matryoshka_ln", ctypes.c_int), ("q8", ctypes.c_int)]


class Model:
    """Oracle model built from a pack's config dict and named tensors.

    ``tensors`` maps canonical names to numpy float32 or float16 arrays (f16
    weights are converted exactly, as the reference's raw-mode loader does).
    """

    def __init__(self, cfg: Mapping, tensors: Mapping[str, np.ndarray], q8: bool = False):
        c = _Config()
        c.hidden, c.layers = cfg["hidden_size"], cfg["num_layers"]
        c.heads, c.inter = cfg["num_heads"], cfg["intermediate_size"]
        c.vocab, c.type_vocab = cfg["vocab_size"], cfg.get("type_vocab_size", 0)
        c.max_seq_len, c.max_trained = cfg["max_seq_len"], cfg.get("max_trained_positions", 0) or 0
        c.eps = float(cfg["layer_norm_eps"])
        c.rope = int(cfg["position_encoding"] == "rope")
        c.rope_theta = float(cfg.get("rope_theta", 0.0) or 0.0)
        c.swiglu = int(cfg["activation"] == "swiglu")
        c.pool_cls = int(cfg["pooling"] == "cls")
        c.normalize = int(bool(cfg["normalize"]))
        mat = cfg.get("matryoshka")
        c.matryoshka = int(mat is not None)
        c.matryoshka_ln = int(bool(mat and mat.get("layernorm")))
        c.q8 = int(q8)
        self.cfg = dict(cfg)
        self.hidden = c.hidden
        names = list(tensors)
        arrs = []
        dtypes = []
        for n in names:
            a = tensors[n]
            if a.dtype == np.float16:
                arrs.append(np.ascontiguousarray(a).view(np.uint16))
                dtypes.append(1)
            else:
                arrs.append(np.ascontiguousarray(a, dtype=np.float32))
                dtypes.append(0)
        cnames = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])
        cdata = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
        cdt = (ctypes.c_int * len(names))(*dtypes)
        cnum = (ctypes.c_int64 * len(names))(*[a.size for a in arrs])
        err = ctypes.create_string_buffer(512)
        self._h = lib().fo_model_create(ctypes.byref(c), len(names), cnames, cdata, cdt, cnum, err, 512)
        if not self._h:
            raise ValueError(err.value.decode())

    def close(self):
        if getattr(self, "_h", None):
            lib().fo_model_destroy(self._h)
            self._h = None

    __del__ = close

    def encode(self, ids, out_dim: int = 0) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        n = self.hidden if out_dim == 0 else out_dim
        out = np.zeros(max(n, 1), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        rc = lib().fo_encode(self._h, _ptr(ids), ids.size, out_dim, _ptr(out), err, 512)
        if rc != 0:
            raise ValueError(err.value.decode())
        return out[:n]

    def encode_batch(self, ids: np.ndarray, offsets: np.ndarray, out_dim: int = 0,
                     threads: int = 1) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        offsets = np.ascontiguousarray(offsets, dtype=np.int32)
        nseq = offsets.size - 1
        n = self.hidden if out_dim == 0 else out_dim
        out = np.zeros((nseq, n), dtype=np.float32)
        err = ctypes.create_string_buffer(512)
        rc = lib().fo_encode_batch(self._h, _ptr(ids), _ptr(offsets), nseq, out_dim, _ptr(out), threads,
                                   err, 512)
        if rc != 0:
            raise ValueError(err.value.decode())
        return out
