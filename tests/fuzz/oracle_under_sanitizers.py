"""Runs the oracle's C forward (a sanitizer build selected by
FUTON_ORACLE_LIB) over the reference's toy goldens, fp32 and Q8, single
sequences and batches on 1, 4 and 8 threads (8 > batch: the per-GEMM
threading path).  Launched by tests/test_sanitize.py under
AddressSanitizer + UndefinedBehaviorSanitizer."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))
import oracle  # noqa: E402
import packio  # noqa: E402

worst = 1.0
for pack in ("toy-absolute-gelu", "toy-rope-swiglu"):
    cfg, tensors = packio.read_pack(os.path.join(packio.TOY, pack))
    cases = packio.toy_expected()["packs"][pack]["forward_cases"]
    ids = np.concatenate([np.array(c["ids"], np.int32) for c in cases])
    off = np.concatenate([[0], np.cumsum([len(c["ids"]) for c in cases])]).astype(np.int32)
    for q8 in (False, True):
        m = oracle.Model(cfg, tensors, q8=q8)
        for c in cases:
            v = m.encode(c["ids"])
            if not q8:
                worst = min(worst, packio.cosine(v, c["vector"]))
        for threads in (1, 4, 8):
            m.encode_batch(ids, off, 0, threads=threads)
        m.close()
assert worst >= 0.99999, worst
print(f"oracle under sanitizers: worst cosine vs goldens {worst:.7f}")
