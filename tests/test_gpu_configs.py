"""Parity of the GPU forward with the oracle at each workload's full size,
through the kernels that size actually routes to, and the batch-level
behaviour of fh_encode: length-class scheduling, chunking, cancellation
while the forward executes, stream ordering, fp16 packs.

Gate: every vector at cosine ≥ 0.9999 against the oracle (the restated
reference CPU forward, native/model.go:346-457), as native/parity_test.go:18-21
gates the reference's own kernels."""
import ctypes
import os
import threading
import time

import numpy as np
import pytest

import oracle
import packio
from futon_amd import _lib, synth

pytestmark = pytest.mark.gpu

COS_GATE = 0.9999
THREADS = 16


def _native():
    from futon_amd import native
    return native


def _model(w, tensors=None):
    native = _native()
    if tensors is None:
        tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    return native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8), tensors


def _cos_rows(got, want):
    num = (got.astype(np.float64) * want).sum(1)
    den = np.linalg.norm(got.astype(np.float64), axis=1) * np.linalg.norm(want.astype(np.float64), axis=1)
    return num / den


def _check(name, got, want, what):
    cos = _cos_rows(got, want)
    print(f"{what}: min cos {cos.min():.7f} mean {cos.mean():.7f} over {len(cos)} vectors", flush=True)
    assert cos.min() >= COS_GATE, (name, int(np.argmin(cos)), float(cos.min()))
    return cos


def _batch_from_lens(lens, seed):
    rng = np.random.default_rng(seed)
    seqs = [[101] + list(rng.integers(1000, 30000, L - 2)) + [102] for L in lens]
    offsets = np.concatenate([[0], np.cumsum([len(s) for s in seqs])]).astype(np.int32)
    return np.concatenate(seqs).astype(np.int32), offsets


def test_bench_batch_bge_small_b256():
    """The bench's exact batch (bge-small, B=256, L 16..128, 18048 tokens):
    the persistent ring GEMM (first layer's QKV) and the fused layer tail
    (every other projection) run, and every vector meets the gate.  The
    bench's device-resident entry point gives the same bits."""
    import torch
    w = synth.workload("bge-small")
    m, tensors = _model(w)
    ids, offsets = synth.make_batch(w.ids_seed, 256, 16, 128)
    T = int(offsets[-1])
    assert _lib.load().fh_route_flags(384, 1536, 0, T) & _lib.FH_ROUTE_RING_QKV
    m.profile_reset()
    m.profile_enable(True)
    got = m.EncodePacked(ids, offsets)
    m.profile_enable(False)
    prof = m.profile_read()
    assert prof["mlp_fused"]["launches"] == 11, prof["mlp_fused"]   # layers 0..10; the CLS layer runs compact
    assert prof["gemm_qkv"]["launches"] == 1                         # layer 0 only: the tail writes the rest
    want = oracle.Model(w.config, tensors).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("bge-small", got, want, "bge-small B=256 (bench batch)")
    dev = torch.device("cuda:0")
    d_ids, d_off = torch.from_numpy(ids).to(dev), torch.from_numpy(offsets).to(dev)
    d_out = torch.empty((256, 384), dtype=torch.float32, device=dev)
    m.EncodeDevice(d_ids.data_ptr(), d_off.data_ptr(), 256, T, int(np.diff(offsets).max()), 0, d_out.data_ptr(),
                   torch.cuda.current_stream().cuda_stream, offsets)
    torch.cuda.synchronize()
    assert np.array_equal(d_out.cpu().numpy().view(np.uint32), got.view(np.uint32))
    m.close()


def test_cls_last_layer_fused_at_large_batch():
    """With ≥ 1921 CLS-pooled sequences the last layer's compact M = nseq
    rows are enough for the fused layer tail too; it must read the compact
    CLS attention rows.  Every vector against the oracle."""
    w = synth.workload("bge-small")
    m, tensors = _model(w)
    ids, offsets = synth.make_batch(w.ids_seed + 11, 2048, 8, 16)
    assert _lib.load().fh_route_flags(384, 1536, 0, 2048) & _lib.FH_ROUTE_MLP
    m.profile_reset()
    m.profile_enable(True)
    got = m.EncodePacked(ids, offsets)
    m.profile_enable(False)
    assert m.profile_read()["mlp_fused"]["launches"] == 12  # the CLS layer fused as well
    want = oracle.Model(w.config, tensors).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("bge-small", got, want, "bge-small B=2048 L 8..16 (CLS layer fused)")
    m.close()


def test_minilm_full_batch():
    w = synth.workload("minilm-l6")
    m, tensors = _model(w)
    ids, offsets = synth.make_batch(w.ids_seed, w.batch, w.len_lo, w.len_hi)
    got = m.EncodePacked(ids, offsets)
    want = oracle.Model(w.config, tensors).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("minilm-l6", got, want, f"minilm-l6 B={w.batch}")
    m.close()


def test_q8_full_batch():
    """bge-small Q8 at its full batch (B=1024, L 8..64): int8 codes and the
    int32 dot are exact, so the margin is set by upstream rounding."""
    w = synth.workload("bge-small-q8")
    m, tensors = _model(w)
    ids, offsets = synth.make_batch(w.ids_seed, w.batch, w.len_lo, w.len_hi)
    got = m.EncodePacked(ids, offsets)
    want = oracle.Model(w.config, tensors, q8=True).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("bge-small-q8", got, want, f"bge-small-q8 B={w.batch}")
    m.close()


def test_bert_base_ring_routed():
    """BERT-base at 8 × 512 tokens: enough rows for every projection to run
    on the ring GEMM (at H=768 the layer tail is not fused)."""
    w = synth.workload("bert-base")
    m, tensors = _model(w)
    ids, offsets = synth.make_batch(w.ids_seed, 8, 512, 512)
    f = _lib.load().fh_route_flags(768, 3072, 0, int(offsets[-1]))
    assert f & 15 == 15, f
    got = m.EncodePacked(ids, offsets)
    want = oracle.Model(w.config, tensors).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("bert-base", got, want, "bert-base B=8 L=512 (ring GEMMs)")
    m.close()


def test_nomic_2048_tokens():
    """nomic-bert (RoPE θ=1000, SwiGLU, Matryoshka 256) with a sequence at the
    full 2048-token context: the multi-block attention accumulates binary16
    probabilities over 32 key blocks."""
    w = synth.workload("nomic-bert")
    m, tensors = _model(w)
    ids, offsets = _batch_from_lens([2048, 1300], 7)
    got = m.EncodePacked(ids, offsets, w.out_dim)
    want = oracle.Model(w.config, tensors).encode_batch(ids, offsets, w.out_dim, threads=THREADS)
    _check("nomic-bert", got, want, "nomic-bert L=[2048,1300] Matryoshka 256")
    m.close()


def test_mixed_lengths_scheduled_by_class():
    """A batch mixing short (≤ 128-token) and long sequences runs sorted
    longest first, with attention launched once per length class: every
    vector equals its single-sequence forward bit for bit
    (native/model_test.go:165-197), in any batch order, and meets the gate
    against the oracle."""
    w = synth.workload("minilm-l6")
    m, tensors = _model(w)
    rng = np.random.default_rng(21)
    lens = list(rng.integers(2, 513, 40)) + [2, 128, 129, 512]
    ids, offsets = _batch_from_lens(lens, 22)
    got = m.EncodePacked(ids, offsets)
    want = oracle.Model(w.config, tensors).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("minilm-l6", got, want, "minilm-l6 mixed L 2..512")
    for i in [0, 5, len(lens) - 4, len(lens) - 3, len(lens) - 2, len(lens) - 1]:
        single = m.EncodePacked(ids[offsets[i]:offsets[i + 1]], np.array([0, lens[i]], np.int32))
        assert np.array_equal(single[0].view(np.uint32), got[i].view(np.uint32)), (i, lens[i])
    perm = rng.permutation(len(lens))
    seqs = [ids[offsets[i]:offsets[i + 1]] for i in perm]
    got2 = m.EncodeBatch(seqs)
    assert np.array_equal(got2.view(np.uint32), got[perm].view(np.uint32))
    m.close()


def test_chunked_batch_equals_whole(monkeypatch):
    """A batch cut into token-capped chunks (FUTON_CHUNK_TOKENS) returns the
    same bits as one chunk."""
    w = synth.workload("bge-small")
    whole, tensors = _model(w)
    monkeypatch.setenv("FUTON_CHUNK_TOKENS", "700")
    chunked, _ = _model(w, tensors)
    ids, offsets = synth.make_batch(w.ids_seed + 3, 96, 2, 200)
    a = whole.EncodePacked(ids, offsets)
    chunked.profile_reset()
    chunked.profile_enable(True)
    b = chunked.EncodePacked(ids, offsets)
    chunked.profile_enable(False)
    assert chunked.profile_read()["pool_l2"]["launches"] > 2  # several forwards
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    whole.close()
    chunked.close()


def test_cancel_observed_while_executing():
    """A cancel flag raised while the forward is already running on the GPU
    (long after every kernel of an unpaced forward would have been enqueued)
    aborts with FH_ECANCELED and leaves out untouched (model.go:400, :603
    check between layers as they run)."""
    w = synth.workload("bge-small")
    m, _ = _model(w)
    ids, offsets = synth.make_batch(w.ids_seed + 5, 4096, 16, 128)
    nseq = offsets.size - 1
    t0 = time.perf_counter()
    m.EncodePacked(ids, offsets)
    dt = time.perf_counter() - t0  # a warm forward, including host copies
    t0 = time.perf_counter()
    m.EncodePacked(ids, offsets)
    dt = min(dt, time.perf_counter() - t0)
    L = _lib.load()
    out = np.full((nseq, 384), 7.0, dtype=np.float32)
    flag = ctypes.c_int32(0)
    res = {}

    def run():
        res["rc"] = L.fh_encode(m.handle, ids.ctypes.data, offsets.ctypes.data, nseq, 0, out.ctypes.data,
                                ctypes.addressof(flag))

    th = threading.Thread(target=run)
    th.start()
    time.sleep(dt * 0.3)
    flag.value = 1
    th.join()
    print(f"forward {dt * 1e3:.1f} ms; rc {res['rc']}", flush=True)
    assert res["rc"] == _lib.FH_ECANCELED
    assert (out == 7.0).all()
    # the model is usable afterwards, with and without a (clear) flag
    flag.value = 0
    a = m.EncodePacked(ids[:offsets[8]], offsets[:9], cancel=flag)
    b = m.EncodePacked(ids[:offsets[8]], offsets[:9])
    assert np.array_equal(a, b)
    m.close()


def test_device_entry_ordered_against_host_entry():
    """fh_encode_device on a caller's stream and fh_encode on the model's own
    stream share the workspace: calls alternating between them, with the
    workspace grown in between, give the bits of separate calls."""
    import torch
    w = synth.workload("bge-small")
    m, _ = _model(w)
    ids_s, off_s = synth.make_batch(w.ids_seed + 1, 64, 16, 64)
    ids_l, off_l = synth.make_batch(w.ids_seed + 2, 512, 16, 128)
    want_s = m.EncodePacked(ids_s, off_s)
    dev = torch.device("cuda:0")
    side = torch.cuda.Stream()
    d_ids, d_off = torch.from_numpy(ids_l).to(dev), torch.from_numpy(off_l).to(dev)
    d_out = torch.empty((512, 384), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        m.EncodeDevice(d_ids.data_ptr(), d_off.data_ptr(), 512, int(off_l[-1]), int(np.diff(off_l).max()), 0,
                       d_out.data_ptr(), side.cuda_stream, off_l)
    got_s = m.EncodePacked(ids_s, off_s)  # queued behind the device call, workspace already grown
    side.synchronize()
    want_l = m.EncodePacked(ids_l, off_l)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(d_out.cpu().numpy().view(np.uint32), want_l.view(np.uint32))
    m.close()


def test_fp16_pack_on_device(tmp_path):
    """Production packs are binary16 (native/kernel.go:37-42,
    safetensors.go:91-97).  An F16 pack and an F32 pack holding the same
    (binary16-representable) values load to the same device weights, so
    their vectors are bit-identical; both meet the gate against the oracle
    reading the F16 pack through the exact f16ToF32."""
    native = _native()
    w = synth.workload("minilm-l6")
    t32 = synth.make_tensors(w.config, w.weight_seed)
    t16 = {k: v.astype(np.float16) for k, v in t32.items()}
    t32r = {k: v.astype(np.float32) for k, v in t16.items()}  # the binary16 values, exactly, as F32
    vocab = os.path.join(packio.GOLDEN, "vocab_bert_uncased.txt")
    d16 = synth.write_pack(str(tmp_path / "p16"), w.config, t16, vocab, dtype="F16")
    d32 = synth.write_pack(str(tmp_path / "p32"), w.config, t32r, vocab, dtype="F32")
    raw = native.LoadSafetensorsRaw(os.path.join(d16, "model.safetensors"))
    assert all(np.asarray(v).dtype == np.float16 for v in raw.values())
    m16, m32 = native.LoadModel(d16), native.LoadModel(d32)
    ids, offsets = synth.make_batch(w.ids_seed, w.batch, w.len_lo, w.len_hi)
    a, b = m16.EncodePacked(ids, offsets), m32.EncodePacked(ids, offsets)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = oracle.Model(w.config, t32r).encode_batch(ids, offsets, 0, threads=THREADS)
    _check("minilm-l6", a, want, "minilm-l6 F16 pack")
    m16.close()
    m32.close()


def _stress_tensors(w, seed=77):
    """bge-small-shaped weights with the features of real BERT checkpoints
    that synthetic N(0, 0.02) weights lack: a few outlier channels with
    large LayerNorm γ and β (every norm), so the residual stream carries
    channels 10-30x larger than the rest; an embedding DC offset (every
    token shares a large per-channel vector), so rows have a mean far from
    zero; larger attention/FFN weights (std 0.05)."""
    t = synth.make_tensors(w.config, w.weight_seed + seed, std=0.05)
    rng = np.random.default_rng(seed)
    H = w.config["hidden_size"]
    out_ch = rng.choice(H, 4, replace=False)
    for name in list(t):
        if name.endswith("norm.weight") or name.endswith("norm1.weight") or name.endswith("norm2.weight"):
            t[name][out_ch] = np.float32([12.0, -9.0, 20.0, 7.5])
        if name.endswith("norm.bias") or name.endswith("norm1.bias") or name.endswith("norm2.bias"):
            t[name][out_ch] = np.float32([3.0, -2.5, 5.0, 1.5])
    dc = (rng.standard_normal(H) * 0.5).astype(np.float32)
    dc[out_ch] += np.float32([4.0, -3.0, 6.0, 2.0])
    t["embeddings.word"] = (t["embeddings.word"] + dc).astype(np.float32)
    return t, out_ch


def test_stress_pack_outlier_channels():
    """The binary16 residual stream and the LayerNorm fold
    (rstd·(y·W'ᵀ − mean·c1) + c2) against the oracle on a pack with outlier
    channels and a DC offset, at the bench's kernel routing (ring GEMM +
    fused layer tail) and at a small batch (tiled GEMMs)."""
    w = synth.workload("bge-small")
    tensors, out_ch = _stress_tensors(w)
    m, _ = _model(w, tensors)
    om = oracle.Model(w.config, tensors)
    keep = np.setdiff1d(np.arange(w.config["hidden_size"]), out_ch)
    for B, seed in ((192, 31), (12, 32)):
        ids, offsets = synth.make_batch(w.ids_seed + seed, B, 16, 128)
        got = m.EncodePacked(ids, offsets)
        want = om.encode_batch(ids, offsets, 0, threads=THREADS)
        _check("bge-small-stress", got, want, f"bge-small stress pack (outlier channels, DC offset) B={B}")
        # the outlier channels dominate the pooled vector: the rest must meet
        # the gate on its own
        _check("bge-small-stress", got[:, keep], want[:, keep], f"  same, the {keep.size} non-outlier channels")
    m.close()
