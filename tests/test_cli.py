"""The `futon embed` command on the MI355X path (futon_amd/futon_embed,
cmd/futon/main.go:68-111): flags, stdin, JSON output, exit codes."""
import json
import os
import subprocess

import numpy as np
import pytest

import packio

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "futon_amd", "futon_embed")

needs_cli = pytest.mark.skipif(not os.path.exists(CLI), reason="futon_embed not built")


def run(args, stdin=""):
    return subprocess.run([CLI, *args], input=stdin, capture_output=True, text=True, timeout=300)


@needs_cli
def test_flag_errors_and_empty_input():
    r = run(["-bogus", "x"])
    assert r.returncode == 2 and "flag provided but not defined: -bogus" in r.stderr
    r = run(["-dims", "abc", "x"])
    assert r.returncode == 2 and "invalid value" in r.stderr
    r = run([], stdin="")
    assert r.returncode == 1 and r.stderr.strip() == "futon: no text to embed"
    r = run(["-models-dir", "/nonexistent", "-model", "x", "hello"])
    assert r.returncode == 1 and r.stderr.startswith("futon: ")


@needs_cli
@pytest.mark.gpu
def test_embed_matches_provider_bitwise():
    """Each output line is one JSON array whose float32 values equal the
    provider's EmbedBatch bit for bit; arguments and stdin lines give the
    same vectors; -dims truncates (Matryoshka pack)."""
    from futon_amd import native
    exp = packio.toy_expected()["packs"]["toy-absolute-gelu"]
    texts = [c["text"] for c in exp["text_cases"]]
    r = run(["-models-dir", packio.TOY, "-model", "toy-absolute-gelu", *texts])
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    assert len(lines) == len(texts)
    got = np.array([json.loads(l) for l in lines], dtype=np.float32)
    want = native.New(os.path.join(packio.TOY, "toy-absolute-gelu")).EmbedBatch(texts)
    assert np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32))
    for g, c in zip(got, exp["text_cases"]):
        assert packio.cosine(g, c["vector"]) >= 0.9999
    r2 = run(["-models-dir", packio.TOY, "-model", "toy-absolute-gelu"], stdin="\n".join(texts) + "\n")
    assert r2.returncode == 0 and r2.stdout == r.stdout
    r3 = run(["-models-dir", packio.TOY, "-model", "toy-rope-swiglu", "-dims", "16", "hello world"])
    assert r3.returncode == 0, r3.stderr
    v = np.array(json.loads(r3.stdout), np.float32)
    assert v.shape == (16,) and abs(float(np.linalg.norm(v)) - 1.0) < 1e-5
