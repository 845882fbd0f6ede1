"""Pins the CPU oracle before it is trusted as the parity target.

Each check is independent of the oracle's own formulas: the reference's
upstream-generated toy goldens (HF BertModel / pinned nomic-bert code), the
reference's error bounds against float64 libm, its f16 known-answer table,
the Q8 closed form in int64, and a float64 GEMM.  A deliberately broken
oracle (a planted mistake) must fail the golden gate."""
import json
import math
import os

import numpy as np
import pytest

import oracle
import packio

TOY_COS, TOY_ABS = 0.99999, 2e-4  # native/model_test.go:19-22


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


@pytest.mark.parametrize("pack", ["toy-absolute-gelu", "toy-rope-swiglu"])
def test_oracle_matches_upstream_toy_goldens(pack):
    exp = packio.toy_expected()["packs"][pack]
    cfg, tensors = packio.read_pack(f"{packio.TOY}/{pack}")
    m = oracle.Model(cfg, tensors)
    cases = exp["forward_cases"] + exp.get("text_cases", [])
    for c in cases:
        got = m.encode(c["ids"])
        assert packio.cosine(got, c["vector"]) >= TOY_COS
        assert np.abs(got - np.asarray(c["vector"])).max() <= TOY_ABS
    for c in exp.get("matryoshka_cases", []):
        got = m.encode(c["ids"], c["dim"])
        assert got.shape == (c["dim"],)
        assert packio.cosine(got, c["vector"]) >= TOY_COS
        assert np.abs(got - np.asarray(c["vector"])).max() <= TOY_ABS


@pytest.mark.parametrize("pack", ["toy-absolute-gelu", "toy-rope-swiglu"])
def test_oracle_q8_toy(pack):
    """native/quant_test.go:152-175: Q8 tracks upstream at cos ≥ 0.98."""
    exp = packio.toy_expected()["packs"][pack]
    cfg, tensors = packio.read_pack(f"{packio.TOY}/{pack}")
    m = oracle.Model(cfg, tensors, q8=True)
    for c in exp["forward_cases"]:
        assert packio.cosine(m.encode(c["ids"]), c["vector"]) >= 0.98


def test_planted_mistakes_fail_the_gate():
    """A dropped type embedding or q/v blocks swapped in the fused QKV weight
    must be caught (the toy's near-uniform attention hides a q↔k swap)."""
    exp = packio.toy_expected()["packs"]["toy-absolute-gelu"]
    cfg, tensors = packio.read_pack(f"{packio.TOY}/toy-absolute-gelu")
    bad = dict(tensors)
    bad["embeddings.token_type"] = np.zeros_like(tensors["embeddings.token_type"])
    m = oracle.Model(cfg, bad)
    c = exp["forward_cases"][1]
    assert np.abs(m.encode(c["ids"]) - np.asarray(c["vector"])).max() > TOY_ABS
    bad = dict(tensors)
    w = tensors["layers.0.attn.qkv.weight"]
    bad["layers.0.attn.qkv.weight"] = np.concatenate([w[64:], w[32:64], w[:32]])  # q ↔ v
    m = oracle.Model(cfg, bad)
    assert packio.cosine(m.encode(c["ids"]), c["vector"]) < TOY_COS


def test_exp_f32_bounds():
    """native/mathf32_test.go:10-27."""
    xs = np.arange(-87.33654 + 0.01, 88.72283 - 0.01, 0.0731, dtype=np.float32)
    worst = 0.0
    for x in xs:
        ref = math.exp(float(x))
        worst = max(worst, abs(oracle.exp_f32(x) - ref) / ref)
    assert worst <= 2 ** -23
    assert oracle.exp_f32(0.0) == 1.0
    assert oracle.exp_f32(-104.0) == 0.0


def test_gelu_and_sigmoid_bounds():
    """native/mathf32_test.go:30-58."""
    worst = 0.0
    for x in np.arange(-12, 12, 0.00917, dtype=np.float32):
        ref = 0.5 * float(x) * (1 + math.erf(float(x) / math.sqrt(2)))
        worst = max(worst, abs(oracle.gelu_f32(x) - ref))
    assert worst <= 1e-6
    for x in (-200.0, 200.0):
        assert oracle.gelu_f32(x) == np.float32(0.5 * x * (1 + math.erf(x / math.sqrt(2))))
    worst = 0.0
    for x in np.arange(-120, 120, 0.0113, dtype=np.float32):
        worst = max(worst, abs(oracle.sigmoid_f32(x) - 1 / (1 + math.exp(-float(x)))))
    assert worst <= 2e-7


def test_f16_known_answers_and_rounding():
    """native/safetensors_test.go:154-207 plus an exhaustive check of every
    binary16 pattern against numpy's IEEE conversion."""
    table = {0x0000: 0.0, 0x3C00: 1.0, 0xBC00: -1.0, 0x4170: 2.71875, 0x0001: 5.960464477539063e-08,
             0x03FF: 6.097555160522461e-05, 0x7BFF: 65504.0}
    for bits, want in table.items():
        assert oracle.f16_to_f32(bits) == want
    assert math.copysign(1, oracle.f16_to_f32(0x8000)) == -1
    assert math.isinf(oracle.f16_to_f32(0x7C00)) and math.isnan(oracle.f16_to_f32(0x7E00))
    allbits = np.arange(0, 1 << 16, 97, dtype=np.uint16)
    ref = allbits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in allbits], np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()
    assert oracle.f16_to_f32(oracle.f32_to_f16(1.0 + 1.0 / 2048)) == 1.0
    assert oracle.f16_to_f32(oracle.f32_to_f16(1.0 + 3.0 / 2048)) == 1.0 + 4.0 / 2048
    assert math.isinf(oracle.f16_to_f32(oracle.f32_to_f16(65520.0)))
    rng = np.random.default_rng(0)
    for v in rng.standard_normal(2000).astype(np.float32) * 100:
        assert oracle.f32_to_f16(float(v)) == int(np.float16(v).view(np.uint16))


def test_q8_quantize_row_invariants():
    """native/quant_test.go:14-52."""
    rng = np.random.default_rng(3)
    src = rng.standard_normal(257).astype(np.float32)
    q, scale = oracle.quantize_row_q8(src)
    amax = float(np.abs(src).max())
    assert scale > 0 and abs(float(scale) - amax / 127) <= 1e-9 * amax
    assert (q != -128).all()
    assert (np.abs(src.astype(np.float64) - q * float(scale)) <= float(scale) / 2 + 1e-7).all()
    q0, s0 = oracle.quantize_row_q8(np.zeros(8, np.float32))
    assert s0 == 0 and not q0.any()


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (2, 3, 7), (4, 4, 8), (5, 9, 16), (7, 16, 33), (13, 29, 65)])
def test_q8_matmul_closed_form(m, n, k):
    """native/quant_test.go:57-100: exact int64 dot of the same codes, one f32 rescale."""
    rng = np.random.default_rng(17 + m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    qb, sb = oracle.quantize_q8(w)
    got = oracle.matmul_t_q8(a, qb, sb, bias)
    for i in range(m):
        qa, sa = oracle.quantize_row_q8(a[i])
        s = qa.astype(np.int64) @ qb.astype(np.int64).T
        want = (s.astype(np.float32) * (np.float32(sa) * sb)).astype(np.float32) + bias
        assert np.array_equal(got[i], want.astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (1, 7, 5), (3, 4, 9), (5, 3, 8), (7, 16, 33), (13, 29, 17),
                                   (32, 6, 100), (37, 203, 300)])
def test_matmul_t_vs_float64(m, n, k):
    """native/kernel_test.go:35-63: float64 naive reference at 1e-4 (1e-3 above 2^21 MACs)."""
    rng = np.random.default_rng(42 + m * n * k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64).T + bias
    tol = 1e-3 if m * n * k >= 1 << 21 else 1e-4
    assert np.abs(oracle.matmul_t(a, b, bias) - want).max() <= tol * max(1.0, math.sqrt(k) / 10)


def test_softmax_and_layernorm_closed_forms():
    row = np.array([1.0, 2.0, 3.0, -200.0], np.float32)
    p = oracle.softmax_scaled(row, 0.5)
    e = np.exp(0.5 * row.astype(np.float64) - 1.5)
    np.testing.assert_allclose(p, e / e.sum(), rtol=2e-7, atol=1e-30)
    assert p[3] == 0.0  # exp argument clamped at -104 flushes to zero
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    y = oracle.layer_norm_rows(x, None, None, 1e-5)
    mu, var = 2.5, 1.25
    np.testing.assert_allclose(y[0], (x[0] - mu) / math.sqrt(var + 1e-5), rtol=1e-6)


def test_encode_rejects_like_reference():
    cfg, tensors = packio.read_pack(f"{packio.TOY}/toy-absolute-gelu")
    m = oracle.Model(cfg, tensors)
    for ids, dim in (([], 0), ([2, 999, 3], 0), ([5] * 65, 0), ([2, 3], 16), ([2, 3], 33)):
        with pytest.raises(ValueError):
            m.encode(ids, dim)


def _bert_shape_cases():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bert_shapes.json")
    with open(path) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("workload", ["minilm-l6", "bge-small", "bert-base"])
def test_oracle_matches_hf_bert_at_real_shapes(workload):
    """The oracle against transformers' BertModel (float64) on the workload's
    own synthetic weights at real widths, heads and depths (fixtures written by
    tests/golden/gen_bert_goldens.py)."""
    from futon_amd import synth
    cases = [c for c in _bert_shape_cases() if c["workload"] == workload]
    assert cases
    w = synth.workload(workload)
    t = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    om = oracle.Model(w.config, t)
    for c in cases:
        got = om.encode(np.array(c["ids"], dtype=np.int32))
        want = np.array(c["vector"])
        cos = float(got @ want / np.linalg.norm(got) / np.linalg.norm(want))
        assert cos >= 0.999999, (workload, len(c["ids"]), cos)
        assert np.abs(got - want).max() < 1e-4
    om.close()
