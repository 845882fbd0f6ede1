"""CPU-side checks of the boundary and the C++ host loader (no GPU compute):
the library loads and exports every function the public headers declare,
creation without a gfx950 device fails loudly, and the pack loader rejects
what the reference's loader rejects (native/model_test.go:479-567,
native/safetensors_test.go:10-152, native/config.go:119-171)."""
import json
import os
import re
import shutil
import struct

import numpy as np
import pytest

import packio
from futon_amd import _lib, native, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in ("futon_hip.h", "futon_hip_ops.h", "futon_host.h"):
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names |= set(re.findall(r"\b(fh_\w+)\s*\(", src))
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    declared = header_functions()
    assert declared == set(_lib.EXPORTED)
    for name in declared:
        assert hasattr(L, name), name


def test_create_without_device_fails_loudly():
    cfg, tensors = packio.read_pack(os.path.join(packio.TOY, "toy-absolute-gelu"))
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    with pytest.raises(_lib.FutonError) as ei:
        native.Model(native.PackConfig.from_dict(cfg), tensors)
    assert ei.value.code == _lib.FH_ENODEV


def copy_pack(tmp_path, name="toy-absolute-gelu"):
    dst = tmp_path / name
    shutil.copytree(os.path.join(packio.TOY, name), dst)
    return str(dst)


def mutate_json(path, fn):
    d = json.load(open(path))
    fn(d)
    open(path, "w").write(json.dumps(d))


def rehash(dir):
    def fn(m):
        for member in m["members"]:
            p = os.path.join(dir, member)
            m["members"][member] = {"sha256": native.sha256_file(p), "size": os.path.getsize(p)}
    mutate_json(os.path.join(dir, "manifest.json"), fn)


def validate_pack(dir):
    """LoadModel up to (not including) the device upload, in the C++ host layer."""
    p = native.LoadPack(dir)
    return p.config, p.tensor_count()


def test_toy_packs_validate():
    for name in ("toy-absolute-gelu", "toy-rope-swiglu"):
        cfg, n = validate_pack(os.path.join(packio.TOY, name))
        assert cfg.EffectiveMaxSeqLen() == 64 and n > 10


@pytest.mark.parametrize("case", ["wrong_format", "prenorm", "edited_config_stale_manifest", "missing_manifest",
                                  "truncated_weights", "removed_bias_rehashed", "bad_theta", "bad_matryoshka",
                                  "string_dim", "mixed_model_id", "stale_tensor_names", "missing_vocab_member"])
def test_pack_tamper_fails_loudly(tmp_path, case):
    d = copy_pack(tmp_path, "toy-rope-swiglu" if case in ("bad_theta", "bad_matryoshka") else "toy-absolute-gelu")
    cfgp = os.path.join(d, "config.json")
    if case == "wrong_format":
        mutate_json(cfgp, lambda m: m.update(pack_format=99))
        rehash(d)
    elif case == "prenorm":
        mutate_json(cfgp, lambda m: m.update(pre_norm=True))
        rehash(d)
    elif case == "edited_config_stale_manifest":
        mutate_json(cfgp, lambda m: m.update(normalize=False))
    elif case == "missing_manifest":
        os.remove(os.path.join(d, "manifest.json"))
    elif case == "truncated_weights":
        p = os.path.join(d, "model.safetensors")
        raw = open(p, "rb").read()
        open(p, "wb").write(raw[:-100])
    elif case == "removed_bias_rehashed":
        p = os.path.join(d, "model.safetensors")
        t = native.LoadSafetensors(p)
        del t["layers.0.attn.qkv.bias"]
        synth.write_safetensors(t, p)
        rehash(d)
    elif case == "bad_theta":
        mutate_json(cfgp, lambda m: m.update(rope_theta=0))
        rehash(d)
    elif case == "bad_matryoshka":
        mutate_json(cfgp, lambda m: m.update(matryoshka={"layernorm": True, "dims": [64]}))
        rehash(d)
    elif case == "string_dim":
        mutate_json(cfgp, lambda m: m.update(hidden_size="32"))
        rehash(d)
    elif case == "mixed_model_id":
        mutate_json(os.path.join(d, "manifest.json"), lambda m: m.update(model_id="other"))
    elif case == "stale_tensor_names":
        mutate_json(os.path.join(d, "manifest.json"), lambda m: m["tensor_names"].append("extra.weight"))
    elif case == "missing_vocab_member":
        mutate_json(os.path.join(d, "manifest.json"), lambda m: m["members"].pop("vocab.txt"))
    with pytest.raises(native.PackError):
        validate_pack(d)


def test_config_decoding_follows_go_json(tmp_path):
    """encoding/json field semantics: unknown members ignored, null leaves a
    field unset, keys match case-insensitively, clamp by max_trained_positions."""
    d = copy_pack(tmp_path, "toy-rope-swiglu")
    cfgp = os.path.join(d, "config.json")

    def edit(m):
        m["unknown_field"] = {"x": [1, 2]}
        m["HIDDEN_SIZE"] = m.pop("hidden_size")
        m["prefixes"] = None
        m["max_trained_positions"] = 16
    mutate_json(cfgp, edit)
    rehash(d)
    cfg, n = validate_pack(d)
    assert cfg.EffectiveMaxSeqLen() == 16 and n > 10


def _st(entries, data):
    hj = json.dumps(entries).encode()
    return struct.pack("<Q", len(hj)) + hj + data


@pytest.mark.parametrize("raw", [
    b"\x01\x02",
    struct.pack("<Q", 1 << 30) + b"{}",
    _st({"a": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4),
    _st({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8),
    _st({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 12),
    _st({"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8),
    _st({"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, b"\0" * 4),
    _st({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
         "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}, b"\0" * 12),
    _st({"a": {"dtype": "F32", "shape": [1 << 32, 1 << 32], "data_offsets": [0, 0]}}, b""),
])
def test_safetensors_rejects_malformed(raw):
    with pytest.raises(native.PackError):
        native.ParseSafetensors(raw)


def test_safetensors_round_trip_f16_raw():
    t = {"w": np.arange(6, dtype=np.float32).reshape(2, 3)}
    import io
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "m.safetensors")
        synth.write_safetensors(t, p, "F16")
        raw = native.LoadSafetensorsRaw(p)
        assert raw["w"].dtype == np.dtype("<f2")
        assert np.array_equal(native.LoadSafetensors(p)["w"], t["w"])
        del io


def test_synthetic_pack_is_deterministic(tmp_path):
    cfg = json.load(open(os.path.join(packio.TOY, "toy-absolute-gelu", "config.json")))
    a = synth.make_tensors(cfg, 7)
    b = synth.make_tensors(cfg, 7)
    for k in a:
        assert np.array_equal(a[k], b[k])
    d = synth.write_pack(str(tmp_path / "p"), cfg, a)
    c2, n2 = validate_pack(d)
    assert c2.model_id == cfg["model_id"] and n2 == len(a)
    ids, off = synth.make_batch(42, 64, 16, 128)
    lens = np.diff(off)
    assert lens.min() >= 16 and lens.max() <= 128
    assert (ids[off[:-1]] == 101).all() and (ids[off[1:] - 1] == 102).all()
    inner = np.delete(ids, np.concatenate([off[:-1], off[1:] - 1]))
    assert inner.min() >= 1000 and inner.max() <= 30521


def test_routing_falls_back_before_32bit_offsets_overflow():
    """The persistent ring GEMM and the fused layer tail address rows with
    32-bit buffer offsets.  At the row counts where those offsets would
    overflow, the forward must route the projection to the tiled GEMM
    (64-bit indices, same bits) instead of failing; below them it keeps the
    fast kernels.  Host-only: fh_route_flags evaluates the same predicates
    run_forward_fold uses."""
    from futon_amd import _lib
    L = _lib.load()
    R = _lib
    all_ring = R.FH_ROUTE_RING_QKV | R.FH_ROUTE_RING_OUT | R.FH_ROUTE_RING_FFN1 | R.FH_ROUTE_RING_FC2
    # bge-small / MiniLM (H=384, I=1536, GELU): everything fused at the bench size
    f = L.fh_route_flags(384, 1536, 0, 18048)
    assert f & all_ring == all_ring and f & R.FH_ROUTE_MLP and f & R.FH_ROUTE_MLP_QKV
    # small batches: tiled GEMMs, nothing fused (fewer than 192 ring tiles)
    assert L.fh_route_flags(384, 1536, 0, 1000) == 0
    # the fused tail's next-layer Q/K/V ([M, 1152] binary16) overflows at M·2304 ≥ 2^31
    lim_q = (1 << 31) // (3 * 384 * 2)
    assert L.fh_route_flags(384, 1536, 0, lim_q) & R.FH_ROUTE_MLP_QKV
    assert not L.fh_route_flags(384, 1536, 0, lim_q + 1) & R.FH_ROUTE_MLP_QKV
    assert L.fh_route_flags(384, 1536, 0, lim_q + 1) & R.FH_ROUTE_MLP
    # the QKV ring GEMM at H=384 writes [M+256, 1152] binary16 rows
    lim = (1 << 31) // (3 * 384 * 2) - 256
    assert L.fh_route_flags(384, 1536, 0, lim - 1) & R.FH_ROUTE_RING_QKV
    assert not L.fh_route_flags(384, 1536, 0, lim + 1) & R.FH_ROUTE_RING_QKV
    # BERT-base FFN1 (ldc = 3072): ring up to (M+256)·6144 < 2^31
    lim = (1 << 31) // (3072 * 2) - 256
    f_ok, f_over = L.fh_route_flags(768, 3072, 0, lim - 1), L.fh_route_flags(768, 3072, 0, lim + 1)
    assert f_ok & R.FH_ROUTE_RING_FFN1 and not f_over & R.FH_ROUTE_RING_FFN1
    assert f_over & R.FH_ROUTE_RING_OUT  # the narrower outputs still fit
    assert not f_ok & R.FH_ROUTE_MLP  # the fused tail is built for hidden 384 only
    # SwiGLU's interleaved FFN1 (N = 2·I, C [M, I]) takes the ring too, to the same row limit;
    # H=32 (toy) is not folded
    assert L.fh_route_flags(768, 3072, 1, lim - 1) & R.FH_ROUTE_RING_FFN1
    assert not L.fh_route_flags(768, 3072, 1, lim + 1) & R.FH_ROUTE_RING_FFN1
    assert L.fh_route_flags(32, 64, 0, 1 << 20) == 0
