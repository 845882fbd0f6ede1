#!/usr/bin/env python3
"""Writes tests/golden/bert_shapes.json: embeddings of a few synthetic
sequences computed by the locally installed transformers BertModel (float64,
eager attention) from the same seeded synthetic weights the workloads use,
at the real BERT-family shapes (MiniLM-L6, bge-small, BERT-base).

This is an independent implementation of the absolute-position + erf-GELU
post-norm encoder the reference runs (native/model.go:346-457); it pins the
oracle and the GPU forward at real widths, head counts and depths, where the
reference's own toy goldens (hidden 32) cannot.  Pooling, Matryoshka and L2
follow native/model.go:417-453.  Run from the repository root:

    python3 tests/golden/gen_bert_goldens.py
"""
import json
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from futon_amd import synth  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bert_shapes.json")
CASES = [("minilm-l6", 4, 8, 40), ("bge-small", 4, 16, 48), ("bert-base", 2, 20, 40)]


def hf_state(cfg, t):
    H = cfg["hidden_size"]
    sd = {
        "embeddings.word_embeddings.weight": t["embeddings.word"],
        "embeddings.position_embeddings.weight": t["embeddings.position"],
        "embeddings.token_type_embeddings.weight": t["embeddings.token_type"],
        "embeddings.LayerNorm.weight": t["embeddings.norm.weight"],
        "embeddings.LayerNorm.bias": t["embeddings.norm.bias"],
    }
    for i in range(cfg["num_layers"]):
        p, q = f"layers.{i}.", f"encoder.layer.{i}."
        w, b = t[p + "attn.qkv.weight"], t[p + "attn.qkv.bias"]
        for j, n in enumerate(("query", "key", "value")):
            sd[q + f"attention.self.{n}.weight"] = w[j * H:(j + 1) * H]
            sd[q + f"attention.self.{n}.bias"] = b[j * H:(j + 1) * H]
        sd[q + "attention.output.dense.weight"] = t[p + "attn.out.weight"]
        sd[q + "attention.output.dense.bias"] = t[p + "attn.out.bias"]
        sd[q + "attention.output.LayerNorm.weight"] = t[p + "norm1.weight"]
        sd[q + "attention.output.LayerNorm.bias"] = t[p + "norm1.bias"]
        sd[q + "intermediate.dense.weight"] = t[p + "mlp.fc1.weight"]
        sd[q + "intermediate.dense.bias"] = t[p + "mlp.fc1.bias"]
        sd[q + "output.dense.weight"] = t[p + "mlp.fc2.weight"]
        sd[q + "output.dense.bias"] = t[p + "mlp.fc2.bias"]
        sd[q + "output.LayerNorm.weight"] = t[p + "norm2.weight"]
        sd[q + "output.LayerNorm.bias"] = t[p + "norm2.bias"]
    return {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in sd.items()}


def main():
    from transformers import BertConfig, BertModel
    out = {"generator": "transformers %s BertModel, float64, eager attention" % __import__("transformers").__version__,
           "cases": []}
    for name, n, lo, hi in CASES:
        w = synth.workload(name)
        cfg = w.config
        t = synth.make_tensors(cfg, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
        bc = BertConfig(vocab_size=cfg["vocab_size"], hidden_size=cfg["hidden_size"],
                        num_hidden_layers=cfg["num_layers"], num_attention_heads=cfg["num_heads"],
                        intermediate_size=cfg["intermediate_size"], max_position_embeddings=cfg["max_seq_len"],
                        type_vocab_size=cfg["type_vocab_size"], layer_norm_eps=cfg["layer_norm_eps"],
                        hidden_act="gelu", attn_implementation="eager")
        m = BertModel(bc, add_pooling_layer=False).double().eval()
        missing, unexpected = m.load_state_dict(hf_state(cfg, t), strict=False)
        assert not unexpected and all("position_ids" in k or "token_type_ids" in k for k in missing), missing
        ids, off = synth.make_batch(w.ids_seed + 1000, n, lo, hi)
        for i in range(n):
            seq = ids[off[i]:off[i + 1]]
            with torch.no_grad():
                h = m(torch.from_numpy(seq.astype(np.int64))[None]).last_hidden_state[0].numpy()
            v = h[0] if cfg["pooling"] == "cls" else h.mean(axis=0)
            if cfg.get("normalize", True):
                v = v / np.linalg.norm(v)
            out["cases"].append({"workload": name, "ids": seq.tolist(), "vector": [float(x) for x in v]})
    with open(OUT, "w") as f:
        json.dump(out, f)
    print(f"wrote {OUT}: {len(out['cases'])} cases")


if __name__ == "__main__":
    main()
