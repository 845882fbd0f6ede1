"""AddressSanitizer + UndefinedBehaviorSanitizer over the code that reads
untrusted bytes on the host and over the oracle:

* the host parsers (safetensors reader, pack-config JSON decoder, WordPiece
  tokenizer; futon_amd/csrc/host/) driven by a seeded fuzz loop
  (tests/fuzz/fuzz_host.cpp), with the reference's tokenizer fuzz properties
  (native/tokenizer_test.go:130-168): never crash, always a well-formed
  [CLS] … [SEP] sequence within bounds, deterministic;
* the oracle's C forward over the toy goldens.

CPU only: the sanitized builds are plain g++/gcc builds of host code, made
in a temporary directory."""
import os
import shutil
import subprocess
import zlib

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "futon_amd", "csrc", "host")
GOLDEN = os.path.join(ROOT, "tests", "golden")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None,
                                reason="needs gcc/g++")


@pytest.fixture(scope="module")
def fuzz_bin(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("san") / "fuzz_host")
    srcs = [os.path.join(ROOT, "tests", "fuzz", "fuzz_host.cpp")] + \
        [os.path.join(HOST, f) for f in ("pack.cpp", "util.cpp", "tokenizer.cpp", "error.cpp")]
    subprocess.run(["g++", "-std=c++17", *SAN, "-I", os.path.join(ROOT, "include"), "-I", HOST, *srcs, "-o", out],
                   check=True)
    return out


@pytest.mark.parametrize("mode,seed_file,iters", [
    ("safetensors", os.path.join(GOLDEN, "toy", "toy-absolute-gelu", "model.safetensors"), 6000),
    ("safetensors", os.path.join(GOLDEN, "toy", "toy-rope-swiglu", "model.safetensors"), 6000),
    ("config", os.path.join(GOLDEN, "toy", "toy-rope-swiglu", "config.json"), 30000),
    ("config", os.path.join(GOLDEN, "toy", "toy-absolute-gelu", "config.json"), 30000),
    ("tokenizer", os.path.join(GOLDEN, "vocab_bert_uncased.txt"), 20000),
])
def test_host_parsers_fuzzed_under_sanitizers(fuzz_bin, mode, seed_file, iters):
    r = subprocess.run([fuzz_bin, mode, seed_file, str(iters), str(zlib.crc32(f"{mode}:{os.path.basename(seed_file)}".encode()) % 1000 + 7)],
                       capture_output=True, text=True, env=ENV, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]


def test_oracle_under_sanitizers(tmp_path):
    lib = str(tmp_path / "liboracle_san.so")
    subprocess.run(["gcc", "-std=c11", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math", "-fPIC",
                    "-fopenmp", *SAN, "-shared", "-o", lib, os.path.join(ROOT, "oracle", "oracle.c"), "-lm"],
                   check=True)
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    ubsan = subprocess.run(["gcc", "-print-file-name=libubsan.so"], capture_output=True, text=True).stdout.strip()
    env = dict(ENV, LD_PRELOAD=f"{asan} {ubsan}", FUTON_ORACLE_LIB=lib)
    r = subprocess.run(["python3", os.path.join(ROOT, "tests", "fuzz", "oracle_under_sanitizers.py")],
                       capture_output=True, text=True, env=env, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
