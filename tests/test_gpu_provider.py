"""Text → vector through the C++ host layer (tokenizer + Provider) and the
GPU forward, mirroring the reference's provider tests
(native/model_test.go:99-120, :160-197, :246-300) and futon.New."""
import ctypes
import json
import os
import shutil

import numpy as np
import pytest

import packio

pytestmark = pytest.mark.gpu

COS_GATE = 0.9999


def _native():
    from futon_amd import native
    return native


def toy_dir(name):
    return os.path.join(packio.TOY, name)


def copy_pack(tmp_path, name):
    dst = tmp_path / name
    shutil.copytree(toy_dir(name), dst)
    return str(dst)


def rehash(dir):
    native = _native()
    mp = os.path.join(dir, "manifest.json")
    m = json.load(open(mp))
    for member in m["members"]:
        p = os.path.join(dir, member)
        m["members"][member] = {"sha256": native.sha256_file(p), "size": os.path.getsize(p)}
    json.dump(m, open(mp, "w"))


def test_toy_provider_end_to_end():
    """TestToyProviderEndToEnd: text cases (empty string and [UNK]-bearing
    text included) against vectors from the HF tokenizer + upstream model."""
    exp = packio.toy_expected()["packs"]["toy-absolute-gelu"]
    assert exp["text_cases"]
    p = _native().New(toy_dir("toy-absolute-gelu"))
    worst = 1.0
    for c in exp["text_cases"]:
        got = p.Embed(c["text"])
        cos = packio.cosine(got, c["vector"])
        worst = min(worst, cos)
        assert cos >= COS_GATE, (c["text"], cos)
        assert np.abs(got - np.array(c["vector"])).max() < 2e-3
    # the same texts in one batch give the same vectors bit for bit
    batch = p.EmbedBatch([c["text"] for c in exp["text_cases"]])
    for i, c in enumerate(exp["text_cases"]):
        assert np.array_equal(batch[i].view(np.uint32), p.Embed(c["text"]).view(np.uint32))
    print(f"provider text cases: min cosine vs upstream {worst:.7f}")


def test_provider_batch_matches_single():
    """TestBatchMatchesSingle (model_test.go:165-197)."""
    p = _native().New(toy_dir("toy-rope-swiglu"))
    texts = ["the cat sat on the mat.", "hello", "", "snowman runs", "the the the the the the the the", "unaffable!"]
    batch = p.EmbedBatch(texts)
    for i, t in enumerate(texts):
        single = p.Embed(t)
        assert single.shape == batch[i].shape
        assert np.array_equal(single.view(np.uint32), batch[i].view(np.uint32)), (i, t)


def test_trained_context_clamp(tmp_path):
    """TestTrainedContextClampToy (model_test.go:246-300)."""
    native = _native()
    d = copy_pack(tmp_path, "toy-rope-swiglu")
    cp = os.path.join(d, "config.json")
    cfg = json.load(open(cp))
    cfg["max_trained_positions"] = 16
    json.dump(cfg, open(cp, "w"))
    rehash(d)
    p = native.New(d)
    tok = native.NewTokenizer(os.path.join(d, "vocab.txt"), cfg["tokenizer"])
    long = "the cat sat on the mat . hello world snow man runs . the cat sat on the mat . hello world"
    assert len(tok.Encode(long, cfg["max_seq_len"])) > 16
    got = p.Embed(long)
    ids16 = tok.Encode(long, 16)
    assert len(ids16) == 16
    m = native.LoadModel(d)
    want = m.EncodeTokens(ids16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(Exception):
        m.EncodeTokens([5] * 17)


def test_provider_dimensions_name_close():
    native = _native()
    p = native.New(toy_dir("toy-rope-swiglu"), dimensions=16)
    assert p.Dimensions() == 16
    assert p.ModelName().startswith("native/")
    exp = packio.toy_expected()["packs"]["toy-rope-swiglu"]
    m = native.LoadModel(toy_dir("toy-rope-swiglu"))
    v = p.Embed("hello world")
    tok = native.NewTokenizer(os.path.join(toy_dir("toy-rope-swiglu"), "vocab.txt"),
                              json.load(open(os.path.join(toy_dir("toy-rope-swiglu"), "config.json")))["tokenizer"])
    assert np.array_equal(v.view(np.uint32), m.EncodeTokens(tok.Encode("hello world", 64), 16).view(np.uint32))
    assert exp["matryoshka_cases"]
    assert p.IsAvailable()
    p.Close()
    p.Close()  # idempotent
    assert not p.IsAvailable()
    with pytest.raises(Exception, match="closed"):
        p.Embed("x")
    with pytest.raises(native.PackError):
        native.New(toy_dir("toy-absolute-gelu"), dimensions=16)  # no Matryoshka support
    with pytest.raises(native.PackError):
        native.New("")


def test_provider_cancellation():
    """A set cancel flag aborts the batch with ECANCELED and no vectors."""
    from futon_amd import _lib
    p = _native().New(toy_dir("toy-absolute-gelu"))
    flag = ctypes.c_int32(1)
    with pytest.raises(_lib.FutonError) as ei:
        p.EmbedBatch(["hello", "world"], cancel=flag)
    assert ei.value.code == _lib.FH_ECANCELED


def test_futon_new_resolves_models_dir(tmp_path):
    """futon.New: ModelsDir/Model resolution and the not-installed error."""
    native = _native()
    shutil.copytree(toy_dir("toy-absolute-gelu"), tmp_path / "toy-absolute-gelu")
    p = native.futon_New(model="toy-absolute-gelu", models_dir=str(tmp_path))
    q = native.New(toy_dir("toy-absolute-gelu"))
    assert np.array_equal(p.Embed("hello").view(np.uint32), q.Embed("hello").view(np.uint32))
    with pytest.raises(native.PackError, match="not installed"):
        native.futon_New(model="absent-model", models_dir=str(tmp_path))
    with pytest.raises(native.PackError, match="invalid pack id"):
        native.futon_New(model="../x", models_dir=str(tmp_path))
