#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of the MI355X engine (libchpe.so).

Workload: Qwen2.5-3B with 4-bit GROUP128 cells (dense 17408-byte records, the seeded archive
of libchpe_pack.so), KV cache in fp16 in HBM, a 4096-token seeded random prompt decoded
teacher-forced (untimed; it builds the context), then `--steps` greedy decode steps timed
(256 by default: the 256 decoded tokens).  `--warmup` untimed steps run first, at positions
0..W-1 of the same prompt, before the context is built.

A step is one CHPEEngine.forwardDecode (src/chpe_engine.zig:1663-1803): embed, 36 layers,
LM head, argmax, with the argmax fed back on the device.  Inputs are resident in HBM before
the timed region starts.

Printed on stdout: ONE JSON line; diagnostics go to stderr.
  roofline      the kernel that takes the largest share of the step: algorithmic bytes per
                launch / mean launch time, timed with HIP events around every launch of it
                inside real decode steps (chpe_time_stage_live)
  cpu_baseline  the CPU oracle (oracle/, a C restatement of the reference's forwardDecode)
                on the host cores, on a bounded sample of the same workload: decode steps at
                positions 4096.. after a synthetic KV fill of 4096 positions
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "chpe-qwen-engine_amd"))

METRIC = "batch-1 decode tok/s at 1 MI355X; achieved HBM GB/s as % of peak"
PEAK_HBM_GBS = 8000.0
V, D, LAYERS, KV_HEADS, HEAD_DIM, Q_HEADS = 151936, 2048, 36, 2, 128, 16
ATTN_CHUNK = 8192 // HEAD_DIM  # positions per attention workgroup
NS = "chpe::(anonymous namespace)::"
STAGES = {  # stage id -> (description, kernel name as rocprofv3 prints it, launches per step)
    0: ("q/k/v GEMV + RoPE + KV append (RMSNorm fused)", f"void {NS}k_gemv_mma<4, 1>(chpe::GemvArgs)", LAYERS),
    1: ("o GEMV + residual", f"void {NS}k_gemv_mma<1, 1>(chpe::GemvArgs)", LAYERS),
    2: ("gate/up GEMV + SwiGLU (RMSNorm fused)", f"void {NS}k_gemv_mma<2, 2>(chpe::GemvArgs)", LAYERS),
    3: ("down GEMV + residual (flat tiles)", f"void {NS}k_gemv_flat<1, 3, false, 8>(chpe::GemvArgs)", LAYERS),
    4: ("LM head GEMV + argmax partials", f"{NS}k_gemv_mma_logits(chpe::GemvArgs)", 1),
    5: ("attention over the context chunks", f"void {NS}k_attn_mfma<128, 8, 4, 1>(chpe::AttnArgs)", LAYERS),
    6: ("attention chunk merge", f"void {NS}k_attn_merge<128>(chpe::AttnArgs)", LAYERS),
}



def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attention_bytes(stage, pos):
    """Algorithmic HBM bytes of one attention launch at position `pos` (fp16 KV)."""
    if stage == 5:  # K and V rows 0..pos of one layer, plus q/k/v in and the partials out
        chunks = math.ceil((pos + 1) / ATTN_CHUNK)
        return 2 * KV_HEADS * HEAD_DIM * 2 * (pos + 1) + Q_HEADS * chunks * (HEAD_DIM + 2) * 4
    chunks = math.ceil((pos + 1) / ATTN_CHUNK)
    return Q_HEADS * chunks * (HEAD_DIM + 2) * 4 + Q_HEADS * HEAD_DIM * 4


def traffic_for(stage):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    the copy-kernel factor), committed in profiles/traffic.json; None when not measured."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    t = json.loads(f.read_text()).get(str(stage))
    return None if t is None else t.get("bytes_per_launch")


def cpu_baseline(archive, prompt_len, budget_s, max_steps):
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc
    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "16") or 16))
    o = orc.Oracle(archive, arch=0, max_seq_len=prompt_len + max_steps + 1, kv_f16=True, threads=cores)
    try:
        o.prefill_synthetic(prompt_len, seed=1)
        tok, n, t0 = 151643, 0, time.perf_counter()
        while n < max_steps and time.perf_counter() - t0 < budget_s:
            tok = o.forward(tok, prompt_len + n).argmax_token
            n += 1
        dt = time.perf_counter() - t0
    finally:
        o.close()
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode steps at positions {prompt_len}..{prompt_len + n - 1} of the "
                      f"same archive after a synthetic fp16 KV fill of {prompt_len} positions "
                      f"(oracle/chpe_oracle.c, {cores} threads, {dt:.1f} s)"}


def copy_probe():
    """A plain copy kernel of known size: 4 x 256 MiB device-to-device."""
    import torch
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_per_copy": n, "copies": 4}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--live-steps", type=int, default=4, help="decode steps per stage timing")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU oracle sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 256 MiB device-to-device 4 times (calibrates rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE against known bytes)")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the decode path runs "
              "on a single MI355X; multi-GPU sharding is not built)", file=sys.stderr)
        sys.exit(2)
    if os.environ.get("WORLD_SIZE", "1") != "1":
        print("bench.py is single-process; do not launch it under torch.distributed", file=sys.stderr)
        sys.exit(2)

    import chpe_amd as ca
    try:
        import torch
        device_sync = torch.cuda.synchronize if torch.cuda.is_available() else (lambda: None)
    except ImportError:
        device_sync = lambda: None  # noqa: E731

    t = time.perf_counter()
    archive = ca.ensure_archive(ca.PACK_3B_W4, seed=0)
    log(f"archive {archive} ({archive.stat().st_size / 1e9:.3f} GB) ready in {time.perf_counter() - t:.1f} s")
    P, K, W = args.prompt, args.steps, args.warmup
    max_seq = P + K + 7 * args.live_steps + 8
    e = ca.Engine(archive, arch=0, max_seq_len=max_seq, kv_f16=True)
    prompt = np.random.default_rng(1).integers(0, V, P).astype(np.uint32)

    if W:
        e.generate(prompt[:W], 1)  # W steps at positions 0..W-1
    t = time.perf_counter()
    first = e.generate(prompt, 1)  # teacher-forced context: positions 0..P-1
    prefill_s = time.perf_counter() - t
    log(f"context: {P} teacher-forced steps in {prefill_s:.2f} s ({prefill_s / P * 1e3:.3f} ms/step), "
        f"first generated token {int(first[0])}")

    device_sync()
    t0 = time.perf_counter()
    event_ms = e.time_steps(K)  # K graph launches at positions P..P+K-1, greedy on the device
    device_sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall / K * 1e3
    value = K / wall
    step_bytes = float(np.mean([e.step_bytes(P + i) for i in range(0, K, max(1, K // 16))]))
    log(f"decode: {K} steps {wall * 1e3:.1f} ms wall ({event_ms:.1f} ms events) -> {value:.1f} tok/s, "
        f"{ms_per_step:.4f} ms/step; {step_bytes / 1e9:.4f} GB/step -> "
        f"{step_bytes / (wall / K) / 1e9:.1f} GB/s ({step_bytes / (wall / K) / 1e9 / PEAK_HBM_GBS:.1%} of HBM peak)")

    # per-stage mean launch time inside real decode steps
    stages, pos = {}, P + K
    for st in STAGES:
        avg_ms = e.time_stage_live(st, args.live_steps)
        mid = pos + (args.live_steps - 1) / 2.0
        if st in (5, 6):
            nbytes = attention_bytes(st, mid)
        else:
            nbytes = float(np.mean([e.stage_bytes(st, l) for l in range(1 if st == 4 else LAYERS)]))
        desc, kname, per_step = STAGES[st]
        stages[st] = dict(desc=desc, kernel=kname, us=avg_ms * 1e3, bytes=nbytes, per_step=per_step,
                          share=avg_ms * per_step / ms_per_step)
        log(f"  stage {st} {desc:42s} {avg_ms * 1e3:8.2f} us/launch x{per_step:3d} = "
            f"{avg_ms * per_step:6.3f} ms/step ({stages[st]['share']:.1%}); {nbytes / 1e6:8.3f} MB/launch "
            f"-> {nbytes / avg_ms / 1e6:7.1f} GB/s")
        pos += args.live_steps
    dom = max(stages, key=lambda s: stages[s]["us"] * stages[s]["per_step"])
    d = stages[dom]
    achieved = d["bytes"] / (d["us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic_for(dom),
                "kernel": d["kernel"], "stage": d["desc"], "bytes_per_launch": round(d["bytes"]),
                "us_per_launch": round(d["us"], 3), "share_of_step": round(d["share"], 4)}
    e.close()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(archive, P, args.cpu_budget, 256)
        log(f"cpu baseline: {cpu['value']} tok/s ({cpu['sample']})")

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "Qwen2.5-3B 4-bit GROUP128 cells (dense 17408 B records), "
                               f"{P}-token prompt + {K} greedy decode steps, fp16 KV cache",
                   "prompt_tokens": P, "decode_tokens": K, "batch": 1, "kv_cache": "fp16",
                   "weights": "seeded N(0,0.02) fp16 quantized to 4-bit (libchpe_pack.so, seed 0)",
                   "parallelism": "none (1 GPU)"},
        "step_roofline": {"bytes_per_step": round(step_bytes), "achieved": round(step_bytes / (wall / K) / 1e9, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(step_bytes / (wall / K) / 1e9 / PEAK_HBM_GBS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "context_build_s": round(prefill_s, 3),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
