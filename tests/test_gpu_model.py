"""End-to-end parity of the GPU forward (fh_encode through the C ABI) with the
reference's toy goldens and with the oracle, plus the reference's
behavioural pins: batch ≡ single, determinism, cancellation, rejections."""
import ctypes
import os

import numpy as np
import pytest

import oracle
import packio
from futon_amd import synth

pytestmark = pytest.mark.gpu

COS_GATE = 0.9999  # every vector vs the reference path


def _native():
    from futon_amd import native
    return native


def toy_model(pack, q8=False):
    return _native().LoadModel(os.path.join(packio.TOY, pack), q8=q8)


@pytest.mark.parametrize("pack", ["toy-absolute-gelu", "toy-rope-swiglu"])
def test_toy_forward_matches_upstream_goldens(pack):
    """native/model_test.go:72-97 on the GPU: upstream-generated vectors."""
    exp = packio.toy_expected()["packs"][pack]
    m = toy_model(pack)
    worst = 1.0
    for c in exp["forward_cases"]:
        got = m.EncodeTokens(c["ids"])
        cos = packio.cosine(got, c["vector"])
        worst = min(worst, cos)
        assert cos >= COS_GATE, (pack, len(c["ids"]), cos)
        assert np.abs(got - np.array(c["vector"])).max() < 2e-3
    for c in exp.get("matryoshka_cases", []):
        got = m.EncodeTokens(c["ids"], c["dim"])
        assert got.shape == (c["dim"],)
        assert packio.cosine(got, c["vector"]) >= COS_GATE
    print(f"{pack}: min cosine vs upstream {worst:.7f}")


@pytest.mark.parametrize("pack", ["toy-absolute-gelu", "toy-rope-swiglu"])
def test_toy_q8_forward(pack):
    """native/quant_test.go:152-175 (cos ≥ 0.98 vs upstream) and the oracle's Q8 path at the gate."""
    exp = packio.toy_expected()["packs"][pack]
    cfg, tensors = packio.read_pack(os.path.join(packio.TOY, pack))
    om = oracle.Model(cfg, tensors, q8=True)
    m = toy_model(pack, q8=True)
    for c in exp["forward_cases"]:
        got = m.EncodeTokens(c["ids"])
        assert packio.cosine(got, c["vector"]) >= 0.98
        assert packio.cosine(got, om.encode(c["ids"])) >= COS_GATE


def test_toy_batch_equals_single_bitwise():
    """native/model_test.go:165-197: a batched forward is bit-identical to
    per-sequence forwards, whatever else is in the batch."""
    m = toy_model("toy-rope-swiglu")
    rng = np.random.default_rng(3)
    seqs = [[2] + list(rng.integers(5, 60, n)) + [3] for n in (0, 1, 7, 30, 62, 13)]
    batch = m.EncodeBatch(seqs)
    for i, s in enumerate(seqs):
        single = m.EncodeTokens(s)
        assert np.array_equal(single.view(np.uint32), batch[i].view(np.uint32)), i
    # and in another batch order / composition
    batch2 = m.EncodeBatch(seqs[::-1] + seqs[:2])
    for i, s in enumerate(seqs[::-1]):
        assert np.array_equal(batch2[i].view(np.uint32), batch[len(seqs) - 1 - i].view(np.uint32))


def test_determinism_repeated_runs():
    m = toy_model("toy-rope-swiglu")
    ids = [2, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 3]
    ref = m.EncodeTokens(ids)
    for _ in range(3):
        assert np.array_equal(m.EncodeTokens(ids).view(np.uint32), ref.view(np.uint32))


def test_cancellation_at_every_checkpoint():
    """native/model_test.go:218-244: a cancellation landing on any checkpoint
    aborts with ECANCELED and no vector."""
    from futon_amd import _lib
    m = toy_model("toy-rope-swiglu")
    ids = [2, 5, 6, 7, 8, 9, 10, 11, 12, 13, 3]
    total = m.checkpoints_per_call()
    assert total >= 2 * 2  # per layer + between attention and FFN, 2 layers
    for n in range(total):
        m.debug_cancel_after(n)
        with pytest.raises(_lib.FutonError) as ei:
            m.EncodeTokens(ids)
        assert ei.value.code == _lib.FH_ECANCELED
    m.debug_cancel_after(-1)
    flag = ctypes.c_int32(1)
    with pytest.raises(_lib.FutonError) as ei:
        m.EncodeTokens(ids, cancel=flag)
    assert ei.value.code == _lib.FH_ECANCELED
    assert m.EncodeTokens(ids, cancel=ctypes.c_int32(0)).shape == (32,)


def test_model_rejects():
    """native/model_test.go:416-436."""
    from futon_amd import _lib
    m = toy_model("toy-absolute-gelu")
    for ids, dim, code in [([], 0, _lib.FH_EINVAL), ([2, 999, 3], 0, _lib.FH_EINVAL),
                           ([5] * 65, 0, _lib.FH_ETOOLONG), ([2, 3], 16, _lib.FH_EINVAL),
                           ([2, 3], 33, _lib.FH_EINVAL), ([2, -1, 3], 0, _lib.FH_EINVAL)]:
        with pytest.raises(_lib.FutonError) as ei:
            m.EncodeTokens(ids, dim)
        assert ei.value.code == code, (ids, dim)


def _workload_check(name, batch, max_len=None, len_lo=None, threads=16):
    w = synth.workload(name)
    cfg = w.config
    tensors = synth.make_tensors(cfg, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    lo = len_lo if len_lo is not None else w.len_lo
    hi = max_len if max_len is not None else w.len_hi
    ids, offsets = synth.make_batch(w.ids_seed, batch, lo, hi)
    native = _native()
    m = native.Model(native.PackConfig.from_dict(cfg), tensors, q8=w.q8)
    got = m.EncodePacked(ids, offsets, w.out_dim)
    om = oracle.Model(cfg, tensors, q8=w.q8)
    want = om.encode_batch(ids, offsets, w.out_dim, threads=threads)
    cos = [packio.cosine(got[i], want[i]) for i in range(batch)]
    print(f"{name}: B={batch} min cos {min(cos):.7f} mean {np.mean(cos):.7f}")
    assert min(cos) >= COS_GATE, (name, int(np.argmin(cos)), min(cos))
    return m, ids, offsets, got


@pytest.mark.parametrize("name,batch,hi,lo", [
    ("minilm-l6", 8, None, None),
    ("bge-small", 16, None, None),
    ("bge-small-q8", 24, None, None),
    ("bert-base", 2, None, None),
    ("nomic-bert", 2, 640, 512),
])
def test_workload_matches_oracle(name, batch, hi, lo):
    _workload_check(name, batch, hi, lo)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["minilm-l6", "bge-small", "bert-base"])
def test_gpu_matches_hf_bert_at_real_shapes(name):
    """The HIP forward against transformers' BertModel (float64) at the real
    widths, head counts and depths, one ragged batch of the fixture's
    sequences (tests/golden/bert_shapes.json)."""
    import json
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bert_shapes.json")) as f:
        cases = [c for c in json.load(f)["cases"] if c["workload"] == name]
    w = synth.workload(name)
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    native = _native()
    m = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    got = m.EncodeBatch([c["ids"] for c in cases])
    for g, c in zip(got, cases):
        cos = packio.cosine(g, np.array(c["vector"]))
        print(f"{name}: L={len(c['ids'])} cos {cos:.7f}")
        assert cos >= COS_GATE, (name, len(c["ids"]), cos)
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch", [("minilm-l6", 192), ("bge-small", 192), ("bert-base", 24),
                                        ("nomic-bert", 4), ("bge-small-q8", 256)])
def test_ring_gemm_forward_equals_tiled(name, batch, monkeypatch):
    """The folded binary16 forward returns the same bits whether its
    projections run on the persistent ring GEMM (the default, at these
    5k-13k token batches; BERT-base's QKV and FFN1 and nomic-bert's SwiGLU
    FFN1 on 256×256 tiles; the Q8 path's int8 GEMMs on the ring's int8 form)
    or on the tiled GEMM (FUTON_GEMM_RING=0): same K order, same LayerNorm
    statistics reduction, same epilogue arithmetic.  The CLS-pooled last
    layer (bge-small) runs tiled in both."""
    w = synth.workload(name)
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    ids, offsets = synth.make_batch(w.ids_seed + 7, batch, w.len_lo, w.len_hi)
    native = _native()
    ring = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    monkeypatch.setenv("FUTON_GEMM_RING", "0")
    tiled = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    a = ring.EncodePacked(ids, offsets, w.out_dim)
    b = tiled.EncodePacked(ids, offsets, w.out_dim)
    assert np.array_equal(a, b), np.abs(a - b).max()
    ring.close()
    tiled.close()


@pytest.mark.gpu
def test_rope_before_attention_equals_rope_inside(monkeypatch):
    """RoPE packs rotate Q and K once per token before attention (rope_qk);
    the forward returns the same bits as with the rotation inside the
    attention kernels (FUTON_ROPE_QK=0), over both attention classes."""
    w = synth.workload("nomic-bert")
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    parts = [synth.make_batch(w.ids_seed + 11 + i, 1, L, L)[0] for i, L in enumerate((100, 700, 20, 257))]
    ids = np.concatenate(parts).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.int32)
    native = _native()
    pre = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    monkeypatch.setenv("FUTON_ROPE_QK", "0")
    inside = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    a = pre.EncodePacked(ids, offsets, w.out_dim)
    b = inside.EncodePacked(ids, offsets, w.out_dim)
    assert np.array_equal(a, b), np.abs(a - b).max()
    pre.close()
    inside.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,lens,q8", [("minilm-l6", (100, 7, 64, 65, 128, 1), False),
                                          ("nomic-bert", (700, 20, 257, 129), False),
                                          ("bge-small", (100, 7, 128, 1), False), ("bge-small-q8", (60, 9, 33), True),
                                          ("minilm-l6", (90, 5, 129), True)])
def test_ln_pool_matches_separate_layer_norm(name, lens, q8, monkeypatch):
    """Pooling applies the last LayerNorm itself; with FUTON_LN_POOL=0 the
    LayerNorm writes the float32 rows and the pooling reads them back.  Mean
    pooling (fh::ln_pool) adds the same normalized values in another order
    (eight-row groups inside each 64-token segment), so the vectors agree to
    float32 rounding; CLS pooling (fh::ln_cls_pool, binary16 rows or the Q8
    path's float32 rows) gives the same bits.  Batch ≡ single holds.  The
    Q8 path (float32 residual stream) runs both kinds: MiniLM-L6 with Q8
    weights pools by mean from float32 rows."""
    w = synth.workload(name)
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=q8)
    parts = [synth.make_batch(w.ids_seed + 21 + i, 1, L, L)[0] for i, L in enumerate(lens)]
    ids = np.concatenate(parts).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum([len(p) for p in parts])]).astype(np.int32)
    native = _native()
    fused = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=q8)
    monkeypatch.setenv("FUTON_LN_POOL", "0")
    apart = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=q8)
    a = fused.EncodePacked(ids, offsets, w.out_dim)
    b = apart.EncodePacked(ids, offsets, w.out_dim)
    if w.config["pooling"] == "cls":
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.abs(a - b).max()
    assert np.abs(a - b).max() < 2e-6, np.abs(a - b).max()
    cos = np.sum(a * b, axis=1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
    assert cos.min() > 0.9999999, cos.min()
    single = fused.EncodePacked(parts[1], np.array([0, len(parts[1])], dtype=np.int32), w.out_dim)
    assert np.array_equal(single[0].view(np.uint32), a[1].view(np.uint32))
    want = oracle.Model(w.config, tensors, q8=q8).encode_batch(ids, offsets, w.out_dim, threads=16)
    ocos = [packio.cosine(a[i], want[i]) for i in range(len(lens))]
    assert min(ocos) >= COS_GATE, (name, q8, min(ocos))
    fused.close()
    apart.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch", [("minilm-l6", 24), ("bge-small", 300), ("bert-base", 3)])
def test_embedding_statistics_equal_row_stats(name, batch, monkeypatch):
    """The embedding kernel writes the first layer's row statistics itself,
    in row_stats' reduction order over the same binary16 values; the forward
    returns the same bits as with the separate row_stats launch
    (FUTON_EMBED_STATS=0)."""
    w = synth.workload(name)
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    ids, offsets = synth.make_batch(w.ids_seed + 31, batch, w.len_lo, w.len_hi)
    native = _native()
    fused = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    monkeypatch.setenv("FUTON_EMBED_STATS", "0")
    apart = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    a = fused.EncodePacked(ids, offsets, w.out_dim)
    b = apart.EncodePacked(ids, offsets, w.out_dim)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), np.abs(a - b).max()
    fused.close()
    apart.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch", [("minilm-l6", 192), ("bge-small", 192)])
def test_fused_mlp_forward_equals_two_gemms(name, batch, monkeypatch):
    """At hidden width 384 the feed-forward block runs as one fused kernel
    (the default at these 12k-13k token batches); the forward returns the
    same bits as with the block's two ring GEMMs (FUTON_MLP=0)."""
    w = synth.workload(name)
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    ids, offsets = synth.make_batch(w.ids_seed + 9, batch, w.len_lo, w.len_hi)
    native = _native()
    fused = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    monkeypatch.setenv("FUTON_MLP", "0")
    split = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    fused.profile_reset()
    fused.profile_enable(True)
    a = fused.EncodePacked(ids, offsets, w.out_dim)
    fused.profile_enable(False)
    assert fused.profile_read()["mlp_fused"]["launches"] > 0
    b = split.EncodePacked(ids, offsets, w.out_dim)
    assert np.array_equal(a, b), np.abs(a - b).max()
    fused.close()
    split.close()
