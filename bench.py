#!/usr/bin/env python3
"""Throughput of the futon encoder forward on one MI355X.

Workload: bge-small-shaped BERT encoder (12 layers, hidden 384, 12 heads,
FFN 1536, erf-GELU, absolute positions, CLS pooling + L2), fp32 seeded
synthetic weights written as a futon pack and loaded through LoadModel;
batch 256 of [CLS] + Zipf(1.1) ids + [SEP], lengths uniform in 16..128,
packed without padding.  One step = one forward over the whole batch with
ids already resident in HBM (fh_encode_device on torch's current stream).

Prints ONE JSON line: embeddings/s, plus the dominant kernel's roofline
(per-launch algorithmic FLOPs over its HIP-event-timed average duration)
and a CPU baseline (the oracle on the host cores, a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
PEAK_I8_TOPS = 5000.0
PEAK_HBM_GBS = 8000.0
# Every kernel class whose FLOPs are GEMM work: the separate projection GEMMs
# (including the CLS layer's compact ones) and the fused layer tail, which
# is four GEMMs (output projection, FFN1, FC2, next layer's QKV) in one launch.
GEMM_CLASSES = ("gemm_qkv", "gemm_out", "gemm_ffn1", "gemm_fc2", "mlp_fused")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="bge-small")
    ap.add_argument("--pack-root", default=os.path.join(tempfile.gettempdir(), "futon_bench_packs"))
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU-baseline sample time")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mixed", action="store_true",
                    help="instead of the throughput line: a batch of 256 sequences of 2..512 tokens through "
                         "fh_encode, scheduled by attention class (default) against one packed forward "
                         "(FUTON_SCHEDULE=0), host buffers both ways")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (5 launches) and exit; its "
                         "FETCH_SIZE/WRITE_SIZE counters calibrate the per-launch traffic figures")
    return ap.parse_args()


def copy_probe(mib: int) -> None:
    """A plain f32 device-to-device copy of known size, for counter calibration."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "launches": 5}))


def load_traffic(kernel_class: str, workload: str):
    """HBM bytes per launch of `kernel_class` from the committed counter summary
    (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs, each divided by what the same
    counter reads per byte of a plain copy), or None when no summary exists."""
    path = os.path.join(ROOT, "profiles", f"{kernel_class}_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            k, sep, v = line.partition(":")
            if sep and k.strip() in ("fetch_kib_per_dispatch", "write_kib_per_dispatch", "copy_fetch_factor",
                                     "copy_write_factor"):
                vals[k.strip()] = float(v.split()[0])
    if len(vals) != 4:
        return None
    return (vals["fetch_kib_per_dispatch"] / vals["copy_fetch_factor"] +
            vals["write_kib_per_dispatch"] / vals["copy_write_factor"]) * 1024.0


def flops_per_embedding(cfg: dict, L: int) -> float:
    """Algorithmic FLOPs of one unpadded forward (valid tokens only), the
    reference's algorithm including the CLS last-layer shortcut."""
    H, I, N = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_layers"]
    c = 6 if cfg["activation"] == "swiglu" else 4
    full = (8 * H * H + c * H * I) * L + 4 * H * L * L
    if cfg["pooling"] == "cls":
        last = 6 * H * H * L + 4 * H * L + 2 * H * H + c * H * I
        return (N - 1) * full + last
    return N * full


def host_cpus():
    """(usable threads, affinity count, cgroup CPU limit or None, CPU model)."""
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return (min(aff, quota) if quota else aff), aff, quota, model


def cpu_baseline(w, cfg, tensors, ids, offsets, target_s: float):
    """The oracle (the restated reference forward) over a bounded sample of
    the same batch: on every usable host core, one sequence per thread as the
    reference's batchPlan runs large batches, and on one thread."""
    import oracle
    threads, aff, quota, model = host_cpus()
    om = oracle.Model(cfg, tensors, q8=w.q8)
    nseq = offsets.size - 1

    def rate(nthreads, budget):
        # probe on nthreads sequences, then size the sample to ≈ budget seconds
        n0 = min(nseq, nthreads)
        t0 = time.perf_counter()
        om.encode_batch(ids[:offsets[n0]], offsets[:n0 + 1], w.out_dim, nthreads)
        dt = time.perf_counter() - t0
        n = int(min(nseq, max(n0, n0 * budget / max(dt, 1e-3))))
        t0 = time.perf_counter()
        om.encode_batch(ids[:offsets[n]], offsets[:n + 1], w.out_dim, nthreads)
        dt = time.perf_counter() - t0
        return n / dt, n, dt

    v_all, n_all, dt_all = rate(threads, target_s)
    v_one, n_one, dt_one = rate(1, target_s / 2)
    om.close()
    return {"value": round(v_all, 3), "unit": "embeddings/s", "cores": threads, "kind": "port",
            "value_1thread": round(v_one, 3), "nproc": aff, "cgroup_cpu_limit": quota, "cpu_model": model,
            "sample": f"first {n_all} of the {nseq} sequences of the same batch on {threads} threads "
                      f"({dt_all:.2f} s) and the first {n_one} on 1 thread ({dt_one:.2f} s): oracle/oracle.c, "
                      f"the restated reference forward (AVX2-order GEMM), one sequence per thread as the "
                      f"reference's batchPlan at large batch; {aff} CPUs in the affinity mask"
                      + (f", cgroup limit {quota}" if quota else "")}


def mixed_bench(args) -> None:
    """fh_encode over a mixed-length batch: the length-class schedule (one
    forward per attention class, longest first) against one packed forward
    of the whole batch.  Prints one JSON line."""
    from futon_amd import native, synth
    w = synth.workload(args.workload)
    pack = synth.ensure_workload_pack(w, args.pack_root)
    ids, offsets = synth.make_batch(w.ids_seed + 100, 256, 2, 512)
    sched = native.LoadModel(pack, q8=w.q8)
    os.environ["FUTON_SCHEDULE"] = "0"
    try:
        whole = native.LoadModel(pack, q8=w.q8)
    finally:
        del os.environ["FUTON_SCHEDULE"]
    reps = max(5, args.steps // 2)
    res = {}
    for name, m in (("scheduled", sched), ("one_call", whole)):
        for _ in range(3):
            out = m.EncodePacked(ids, offsets, w.out_dim)
        t0 = time.perf_counter()
        for _ in range(reps):
            m.EncodePacked(ids, offsets, w.out_dim)
        res[name] = (offsets.size - 1) * reps / (time.perf_counter() - t0)
        res[name + "_out"] = out
    a, b = res.pop("scheduled_out"), res.pop("one_call_out")
    cos = float(np.min((a.astype(np.float64) * b).sum(1) /
                       (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))))
    lens = np.diff(offsets)
    print(json.dumps({"metric": "mixed-length batch through fh_encode (host buffers), embeddings/s",
                      "workload": f"{w.name}, B=256, L 2..512 (T={int(offsets[-1])}, "
                                  f"{int((lens <= 128).sum())} sequences of <= 128 tokens)",
                      "scheduled": round(res["scheduled"], 1), "one_call": round(res["one_call"], 1),
                      "speedup": round(res["scheduled"] / res["one_call"], 3), "reps": reps,
                      "min_cos_scheduled_vs_one_call": round(cos, 7)}))
    sched.close()
    whole.close()


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are out of scope",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
        return
    if args.mixed:
        mixed_bench(args)
        return
    import torch
    from futon_amd import native, synth

    w = synth.workload(args.workload)
    cfg = w.config
    pack = synth.ensure_workload_pack(w, args.pack_root)
    model = native.LoadModel(pack, q8=w.q8)
    ids, offsets = synth.make_batch(w.ids_seed, w.batch, w.len_lo, w.len_hi)
    lens = np.diff(offsets)
    nseq, T, max_len = int(lens.size), int(offsets[-1]), int(lens.max())
    od = w.out_dim or cfg["hidden_size"]

    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids).to(dev)
    d_off = torch.from_numpy(offsets).to(dev)
    d_out = torch.empty((nseq, od), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def step():
        model.EncodeDevice(d_ids.data_ptr(), d_off.data_ptr(), nseq, T, max_len, w.out_dim, d_out.data_ptr(), sp,
                           offsets)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed * 1e3 / args.steps
    value = nseq * args.steps / elapsed

    # Per-kernel-class HIP-event timing over the same number of steps.
    model.profile_reset()
    model.profile_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    prof = model.profile_read()
    model.profile_enable(False)
    dom = max(prof, key=lambda k: prof[k]["ms"])
    pd = prof[dom]
    per_launch_ms = pd["ms"] / max(pd["launches"], 1)
    traffic = load_traffic(dom, w.name)
    if pd["flops"] > 0:
        peak = PEAK_I8_TOPS if w.q8 and dom.startswith("gemm") else PEAK_F16_TFLOPS
        achieved = pd["flops"] / pd["launches"] / (per_launch_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": traffic,
                "per_launch_flops": pd["flops"] / pd["launches"], "per_launch_bytes": pd["bytes"] / pd["launches"],
                "per_launch_us": round(per_launch_ms * 1e3, 3), "launches_per_step": pd["launches"] // args.steps}
    else:
        achieved = pd["bytes"] / pd["launches"] / (per_launch_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                "per_launch_bytes": pd["bytes"] / pd["launches"], "per_launch_us": round(per_launch_ms * 1e3, 3),
                "launches_per_step": pd["launches"] // args.steps}
    gemm_ms = sum(prof[k]["ms"] for k in GEMM_CLASSES if k in prof)
    gemm_fl = sum(prof[k]["flops"] for k in GEMM_CLASSES if k in prof)
    gemm_tf = gemm_fl / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else 0.0
    total_fl = float(sum(flops_per_embedding(cfg, int(L)) for L in lens))
    kernels = {k: {"ms_per_step": round(v["ms"] / args.steps, 4), "launches_per_step": v["launches"] // args.steps,
                   "tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 1) if v["ms"] and v["flops"] else None,
                   "gbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1) if v["ms"] and v["bytes"] else None}
               for k, v in prof.items() if v["launches"]}

    # End-to-end with host buffers (PCIe-inclusive), reported beside value.
    batch_list = None
    t0 = time.perf_counter()
    reps = max(3, args.steps // 5)
    for _ in range(reps):
        model.EncodePacked(ids, offsets, w.out_dim)
    host_rate = nseq * reps / (time.perf_counter() - t0)
    del batch_list

    result = {
        "metric": "embeddings/sec at 1 MI355X (bge-small, B=256, L<=128); % MFMA peak",
        "value": round(value, 1), "unit": "embeddings/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8" if w.q8 else "f16",
        "data": "synthetic (seeded random-init weights, Zipf ids)",
        "config": {"workload": f"{w.name}: {cfg['num_layers']}L H{cfg['hidden_size']} A{cfg['num_heads']} "
                               f"I{cfg['intermediate_size']} {cfg['activation']} {cfg['pooling']}-pool, "
                               f"B={nseq}, L {w.len_lo}..{w.len_hi} (T={T} tokens, packed)",
                   "global_batch": nseq, "seq_len": max_len, "parallelism": "single-gpu"},
        "roofline": roof,
        "gemm_mfma": {"tflops": round(gemm_tf, 1), "frac": round(gemm_tf / (PEAK_I8_TOPS if w.q8 else PEAK_F16_TFLOPS), 4),
                      "classes": [k for k in GEMM_CLASSES if prof.get(k, {}).get("launches")],
                      "ms_per_step": round(gemm_ms / args.steps, 4)},
        "model_tflops": round(total_fl * value / nseq / 1e12, 1),
        "model_mfma_frac": round(total_fl * value / nseq / 1e12 / (PEAK_I8_TOPS if w.q8 else PEAK_F16_TFLOPS), 4),
        "host_buffers_value": round(host_rate, 1),
        "kernels": kernels,
    }
    if not args.no_cpu:
        tensors = synth.make_tensors(cfg, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
        result["cpu_baseline"] = cpu_baseline(w, cfg, tensors, ids, offsets, args.cpu_seconds)
    model.close()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
