"""Test-side helpers: read a futon pack (config.json + model.safetensors) into
numpy, and the cosine used by the reference's tests (native/util_test.go:13-27)."""
from __future__ import annotations

import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
TOY = os.path.join(GOLDEN, "toy")


def read_safetensors(path: str) -> dict:
    raw = open(path, "rb").read()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + n])
    data = raw[8 + n:]
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        dt = {"F32": np.float32, "F16": np.float16}[e["dtype"]]
        b, en = e["data_offsets"]
        out[name] = np.frombuffer(data[b:en], dtype=dt).reshape(e["shape"]).copy()
    return out


def read_pack(pack_dir: str):
    with open(os.path.join(pack_dir, "config.json")) as f:
        cfg = json.load(f)
    return cfg, read_safetensors(os.path.join(pack_dir, "model.safetensors"))


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        return -2.0
    na, nb = np.sqrt((a * a).sum()), np.sqrt((b * b).sum())
    if na == 0 or nb == 0:
        return -2.0
    return float((a * b).sum() / (na * nb))


def toy_expected() -> dict:
    with open(os.path.join(TOY, "expected.json")) as f:
        return json.load(f)
