#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of the MI355X engine (libchpe.so).

Default workload (--workload qwen72b-w4): Qwen2.5-72B with 4-bit GROUP128 flat tiles (the
seeded archive of libchpe_pack.so, 38.6 GB, resident in HBM), KV cache in fp16 in HBM, an
8192-token seeded random prompt decoded teacher-forced (untimed; it builds the context),
then `--steps` greedy decode steps timed (128 by default).  `--warmup` untimed steps run
first, at positions 0..W-1 of the same prompt, before the context is built.  Other
workloads: qwen72b-w2 (2-bit tiles), qwen3b-w4 (Qwen2.5-3B 4-bit cells, 4096-token prompt),
qwen3b-fp16 (Qwen2.5-3B fp16 raw tiles, 32-token prompt: the reference's own CPU-runnable case),
qwen9b-w4 (Qwen3.5-9B 4-bit flat tiles, the reference's GQA-aliased decode, 2048 tokens),
qwen9b-hybrid (the same archive through the true hybrid layers: gated DeltaNet + gated attention).

A step is one CHPEEngine.forwardDecode (src/chpe_engine.zig:1663-1803): embed, the layers,
LM head, argmax, with the argmax fed back on the device.  Inputs are resident in HBM before
the timed region starts.

Printed on stdout: ONE JSON line; diagnostics go to stderr.
  roofline      the stage (kernel) with the largest share of the step: its algorithmic bytes
                per launch / its mean launch time, timed with HIP events around every launch
                of it inside real decode steps (chpe_time_stage_live)
  cpu_baseline  the CPU oracle (oracle/, a C restatement of the reference's forwardDecode) on
                all of the process's host cores, on a bounded sample of the same workload:
                decode steps after a synthetic fp16 KV fill of the prompt's positions; a
                single-thread figure (the reference's engine is single-threaded) beside it
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
STAGE_DESC = {
    0: "q/k/v GEMV + RoPE + KV append (RMSNorm fused)",
    1: "o GEMV + residual",
    2: "gate/up GEMV + SwiGLU (RMSNorm fused)",
    3: "down GEMV + residual",
    4: "LM head GEMV + argmax partials (final RMSNorm fused)",
    5: "attention over the context chunks",
    6: "attention chunk merge",
}
# per workload: archive kind (chpe_pack.h), architecture, prompt length, shapes
WORKLOADS = {
    "qwen72b-w4": dict(kind=5, arch=2, prompt=8192, V=152064, L=80, H=64, KV=8, hd=128, D=8192, I=29568,
                       desc="Qwen2.5-72B 4-bit GROUP128 flat tiles (dense 17408 B records)"),
    "qwen72b-w2": dict(kind=6, arch=2, prompt=8192, V=152064, L=80, H=64, KV=8, hd=128, D=8192, I=29568,
                       desc="Qwen2.5-72B 2-bit GROUP128 flat tiles (dense 17408 B records)"),
    "qwen3b-w4": dict(kind=2, arch=0, prompt=4096, V=151936, L=36, H=16, KV=2, hd=128, D=2048, I=11008,
                      desc="Qwen2.5-3B 4-bit GROUP128 cells (dense 17408 B records)"),
    "qwen3b-fp16": dict(kind=0, arch=0, prompt=32, V=151936, L=36, H=16, KV=2, hd=128, D=2048, I=11008,
                        desc="Qwen2.5-3B fp16 raw tiles (the reference's own CPU-runnable case)"),
    "qwen9b-w4": dict(kind=7, arch=1, prompt=2048, V=248320, L=32, H=16, KV=4, hd=256, D=4096, I=12288,
                      desc="Qwen3.5-9B 4-bit GROUP128 flat tiles at the INT8 map's indices, "
                           "reference-compatible GQA decode"),
    "qwen9b-hybrid": dict(kind=7, arch=3, oracle_arch=1, hybrid=True, prompt=2048, V=248320, L=32, H=16, KV=4,
                          hd=256, D=4096, I=12288,
                          desc="Qwen3.5-9B 4-bit GROUP128 flat tiles, the true hybrid layers (24 gated "
                               "DeltaNet + 8 gated full attention)"),
}
# the stages both layer kinds of the hybrid model share (its token mixers are timed as the rest)
HYBRID_STAGES = (2, 3, 4)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attention_bytes(w, stage, pos):
    """Algorithmic HBM bytes of one attention launch at position `pos` (fp16 KV); the chunk
    length is the kernels' (attn_chunk_of: 128 positions at head dim 128 with >= 8 kv heads,
    else 8192 / head dim)."""
    chunk = 128 if w["hd"] == 128 and w["KV"] >= 8 else 8192 // w["hd"]
    chunks = math.ceil((pos + 1) / chunk)
    partials = w["H"] * chunks * (w["hd"] + 2) * 4
    if stage == 5:  # K and V rows 0..pos of one layer, the queries in, the partials out
        return 2 * w["KV"] * w["hd"] * 2 * (pos + 1) + w["H"] * w["hd"] * 4 + partials
    return partials + w["H"] * w["hd"] * 4


def traffic_for(workload, stage):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    the copy-kernel factor), committed in profiles/traffic.json; None when not measured."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    t = json.loads(f.read_text()).get(workload, {}).get(str(stage))
    return None if t is None else t.get("bytes_per_launch")


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(archive, w, prompt_len, budget_s):
    """The oracle on the host: all of the process's cores over greedy decode steps at positions
    prompt_len.. after a synthetic fp16 KV fill; then one thread on a sample of one step."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc
    cores = len(os.sched_getaffinity(0))
    o = orc.Oracle(archive, arch=w.get("oracle_arch", w["arch"]), max_seq_len=prompt_len + 64, kv_f16=True,
                   threads=cores)
    try:
        if w.get("hybrid"):
            o.set_hybrid(True)  # (the recurrent states as zero: their cost does not depend on them)
        o.prefill_synthetic(prompt_len, seed=1)
        tok, n, t0 = 151643, 0, time.perf_counter()
        while n < 32 and (n == 0 or time.perf_counter() - t0 < budget_s):
            tok = o.forward(tok, prompt_len + n).argmax_token
            n += 1
        dt = time.perf_counter() - t0
        # one thread: the same step over 0 layers (embedding, final norm, LM head) and over the
        # first layers; per token = t0 + (t_k - t0) * L / k
        o.set_threads(1)
        k = max(1, w["L"] // 10)
        t = time.perf_counter()
        o.forward_layers(tok, prompt_len + n, 0)
        t_head = time.perf_counter() - t
        t = time.perf_counter()
        o.forward_layers(tok, prompt_len + n + 1, k)
        t_k = time.perf_counter() - t
        per_tok_1 = t_head + (t_k - t_head) * w["L"] / k
    finally:
        o.close()
    model = cpu_model()
    return {"value": round(n / dt, 4), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode steps at positions {prompt_len}..{prompt_len + n - 1} of the same "
                      f"archive after a synthetic fp16 KV fill of {prompt_len} positions "
                      f"(oracle/chpe_oracle.c, {cores} threads, {dt:.1f} s) on {model}",
            "cpu_model": model,
            "single_thread": {"value": round(1.0 / per_tok_1, 4), "unit": "tok/s", "cores": 1,
                              "sample": f"one step at position {prompt_len + n + 1} over the first {k} of "
                                        f"{w['L']} layers ({t_k:.2f} s) and over none ({t_head:.2f} s: "
                                        f"embedding, final norm, LM head), scaled to {w['L']} layers"}}


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


def gemv_probe(workload):
    """Only the workload's gate/up GEMV (stage 2: RMSNorm, both projections, SwiGLU) on synthetic
    flat tiles of its shape, 4 launches through the engine's kernel choice for that shape
    (chpe_debug_gemv_flat): the rocprofv3 --pmc traffic runs of the dominant kernel."""
    import chpe_amd as ca
    w = WORKLOADS[workload]
    if w["kind"] not in (5, 6, 7):
        raise SystemExit(f"--gemv-probe: {workload} has no flat-tile gate/up projection")
    bits = 2 if w["kind"] == 6 else 4
    D, I = w["D"], w["I"]
    rng = np.random.default_rng(0)
    tile = ca.pack_flat((rng.standard_normal(32768) * 0.02).astype(np.float32), bits=bits)
    n = (I * D + 32767) // 32768
    gate = np.tile(tile, n)
    up = gate.copy()
    x = rng.standard_normal(D).astype(np.float32)
    g = np.ones(D, np.float32)
    for _ in range(4):
        ca.gpu_gemv_flat("swiglu", I, D, gate, x, tiles_up=up, gamma=g)
    print(json.dumps({"gemv_probe": workload, "rows": I, "cols": D, "bits": bits, "launches": 4}), flush=True)


def stage_probe(workload, iters):
    """The decode step's launches of stages 0 (q/k/v), 1 (o) and 3 (down) alone, `iters` times
    each on layers 0 and 1 of the workload's engine (chpe_time_stage, no context built), then the
    attention kernels (stages 5 and 6) once at the workload's prompt length on synthetic fp16 rows
    (chpe_debug_attention): the rocprofv3 --pmc traffic runs of the stages other than gate/up."""
    import chpe_amd as ca
    w = WORKLOADS[workload]
    archive = ca.ensure_archive(w["kind"], seed=0)
    e = ca.Engine(archive, arch=w["arch"], max_seq_len=64, kv_f16=True)
    try:
        for st in (0, 1, 3):
            e.time_stage(st, 0, 2, iters)
            log(f"stage {st}: {2 * iters} launches")
    finally:
        e.close()
    P = w["prompt"]
    rng = np.random.default_rng(0)
    q = rng.standard_normal(w["H"] * w["hd"]).astype(np.float32)
    k = rng.standard_normal((P + 1, w["KV"] * w["hd"])).astype(np.float32)
    ca.gpu_attention(q, k, k, P, w["H"], w["KV"], w["hd"], 1)
    print(json.dumps({"stage_probe": workload, "stages": [0, 1, 3], "launches_each": 2 * iters,
                      "attention_position": P}), flush=True)


def trace_summary(path, out):
    """Per-kernel statistics of a `rocprofv3 --kernel-trace` CSV (run_kernel_trace.csv) of a
    bench run, split into the decode phase -- the longest run of dispatches without a block-step
    GEMV (k_gemv_mt, k_block_gemm), i.e. the timed decode steps and the stage-timing steps -- and
    the rest (context build, verify, load); block-step kernels are listed per grid shape (one
    shape per projection); writes a Markdown table to `out`."""
    import csv
    import collections
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if "k_block_" in name or "k_gemv_mt" in name:  # block-step launches: by shape (one per projection)
                name += f" grid {r.get('Grid_Size_X', r.get('Grid_Size', '?'))}x{r.get('Grid_Size_Y', '')}"
            rows.append((int(r["Start_Timestamp"]), name, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort()  # (in start order)
    blk = [i for i, r in enumerate(rows) if "k_gemv_mt" in r[1] or "k_block_gemm" in r[1]]
    cuts = [-1] + blk + [len(rows)]
    a, b = max(zip(cuts, cuts[1:]), key=lambda ab: ab[1] - ab[0])
    phases = {"decode": rows[a + 1:b], "other (context build, verify, load)": rows[:a + 1] + rows[b:]}
    lines = [f"Source: `{path}` ({len(rows)} dispatches; decode phase = dispatches {a + 2}..{b} of the run)", ""]
    for name, rs in phases.items():
        st = collections.defaultdict(list)
        for _, k, t0, t1 in rs:
            st[k].append((t1 - t0) / 1e3)
        total = sum(sum(v) for v in st.values()) or 1.0
        lines += [f"### {name}: {len(rs)} dispatches, {total / 1e3:.2f} ms of kernel time", "",
                  "| kernel | calls | avg µs | min µs | max µs | % of phase |", "|---|---|---|---|---|---|"]
        for k, v in sorted(st.items(), key=lambda kv: -sum(kv[1])):
            short = k.replace("chpe::(anonymous namespace)::", "").split("(")[0].replace("void ", "")
            if " grid " in k:
                short += " grid " + k.split(" grid ")[-1]
            lines.append(f"| `{short}` | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                         f"{100 * sum(v) / total:.2f} |")
        lines.append("")
    Path(out).write_text("\n".join(lines))
    print(json.dumps({"trace_summary": str(out), "dispatches": len(rows), "decode": len(phases["decode"])}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="qwen72b-w4", choices=sorted(WORKLOADS))
    ap.add_argument("--prompt", type=int, default=0, help="prompt tokens (default: the workload's)")
    ap.add_argument("--live-steps", type=int, default=2, help="decode steps per stage timing")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU oracle sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 256 MiB device-to-device 4 times (calibrates rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE against known bytes)")
    ap.add_argument("--stage-probe", action="store_true",
                    help="only the q/k/v, o and down launches of layers 0-1 and one attention launch at the "
                         "prompt length (the rocprofv3 --pmc traffic runs of the other stages)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("KERNEL_TRACE_CSV", "OUT_MD"),
                    help="summarise a rocprofv3 kernel-trace CSV of a bench run (decode phase vs the rest) and exit")
    ap.add_argument("--gemv-probe", action="store_true",
                    help="only the workload's gate/up GEMV on synthetic tiles of its shape, 4 launches "
                         "(the rocprofv3 --pmc traffic runs of the dominant kernel)")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.copy_probe:
        copy_probe()
        return
    if args.gemv_probe:
        gemv_probe(args.workload)
        return
    if args.stage_probe:
        stage_probe(args.workload, 2)
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

    w = WORKLOADS[args.workload]
    os.environ.setdefault("CHPE_PACK_PROGRESS", "1")
    t = time.perf_counter()
    archive = ca.ensure_archive(w["kind"], seed=0)
    log(f"archive {archive} ({archive.stat().st_size / 1e9:.3f} GB) ready in {time.perf_counter() - t:.1f} s")
    P, K, W = args.prompt or w["prompt"], args.steps, args.warmup
    max_seq = P + K + 7 * args.live_steps + 16
    t = time.perf_counter()
    e = ca.Engine(archive, arch=w["arch"], max_seq_len=max_seq, kv_f16=True)
    log(f"engine init {time.perf_counter() - t:.1f} s (archive copied to HBM, plans built, step captured)")
    prompt = np.random.default_rng(1).integers(0, w["V"], P).astype(np.uint32)

    if W:
        e.generate(prompt[:W], 1)  # W steps at positions 0..W-1
    block = e.block_ready()
    log(f"building the context: {P} teacher-forced positions "
        f"({'block steps of 32 tokens' if block else 'decode steps'})")
    t = time.perf_counter()
    if block:  # positions 0..P-1, every weight read once per 32 tokens; decode continues from P
        first = [e.prefill(prompt)]
    else:
        first = e.generate(prompt, 1)  # teacher-forced context: positions 0..P-1
    prefill_s = time.perf_counter() - t
    log(f"context: {P} positions in {prefill_s:.2f} s ({P / prefill_s:.1f} tok/s), first generated token {int(first[0])}")

    device_sync()
    t0 = time.perf_counter()
    event_ms = e.time_steps(K)  # K graph launches at positions P..P+K-1, greedy on the device
    device_sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall / K * 1e3
    value = K / wall
    step_bytes = float(np.mean([e.step_bytes(P + i) for i in range(0, K, max(1, K // 16))]))
    log(f"decode: {K} steps {wall * 1e3:.1f} ms wall ({event_ms:.1f} ms events) -> {value:.2f} tok/s, "
        f"{ms_per_step:.4f} ms/step; {step_bytes / 1e9:.4f} GB/step -> "
        f"{step_bytes / (wall / K) / 1e9:.1f} GB/s ({step_bytes / (wall / K) / 1e9 / PEAK_HBM_GBS:.1%} of HBM peak)")

    # per-stage mean launch time inside real decode steps
    stages, pos = {}, P + K
    for st in (HYBRID_STAGES if w.get("hybrid") else STAGE_DESC):
        avg_ms = e.time_stage_live(st, args.live_steps)
        mid = pos + (args.live_steps - 1) / 2.0
        per_step = 1 if st == 4 else w["L"]
        if st in (5, 6):
            nbytes = attention_bytes(w, st, mid)
        else:
            nbytes = float(np.mean([e.stage_bytes(st, l) for l in range(per_step)]))
        stages[st] = dict(desc=STAGE_DESC[st], us=avg_ms * 1e3, bytes=nbytes, per_step=per_step,
                          share=avg_ms * per_step / ms_per_step)
        log(f"  stage {st} {STAGE_DESC[st]:52s} {avg_ms * 1e3:8.2f} us/launch x{per_step:3d} = "
            f"{avg_ms * per_step:6.3f} ms/step ({stages[st]['share']:.1%}); {nbytes / 1e6:9.3f} MB/launch "
            f"-> {nbytes / avg_ms / 1e6:7.1f} GB/s")
        pos += args.live_steps
    if w.get("hybrid"):
        rest = 1.0 - sum(v["share"] for v in stages.values())
        log(f"  the token mixers (DeltaNet and gated attention layers with their projections) and the "
            f"rest: {rest * ms_per_step:.3f} ms/step ({rest:.1%})")
    # batch-M verify: 8 (then 4) drafts at positions pos.. as one block step (or M decode steps)
    drafts = np.random.default_rng(2).integers(0, w["V"], 8).astype(np.uint32)
    verify, by_m = None, {}
    for m in (8, 4):
        e.verify(drafts[:m], pos)
        device_sync()
        reps = 5
        t = time.perf_counter()
        for _ in range(reps):
            e.verify(drafts[:m], pos)
        vt = (time.perf_counter() - t) / reps
        by_m[m] = {"m": m, "ms_per_call": round(vt * 1e3, 3), "positions_per_s": round(m / vt, 2),
                   "vs_batch1_tok_s": round(m / vt / value, 3), "block_step": bool(block), "position": int(pos)}
        log(f"verify: {m} drafts at positions {pos}..{pos + m - 1} in {vt * 1e3:.2f} ms -> {m / vt:.1f} positions/s "
            f"({m / vt / value:.2f}x the batch-1 decode rate; {'one block step' if block else f'{m} decode steps'})")
    verify = dict(by_m[8], m4=by_m[4])
    dom = max(stages, key=lambda s: stages[s]["us"] * stages[s]["per_step"])
    d = stages[dom]
    kernel = e.stage_kernel(dom)
    achieved = d["bytes"] / (d["us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic_for(args.workload, dom),
                "kernel": kernel, "stage": d["desc"], "bytes_per_launch": round(d["bytes"]),
                "us_per_launch": round(d["us"], 3), "share_of_step": round(d["share"], 4)}
    stage_table = {str(s): {"desc": v["desc"], "us_per_launch": round(v["us"], 3), "launches_per_step": v["per_step"],
                            "bytes_per_launch": round(v["bytes"]), "GBps": round(v["bytes"] / v["us"] / 1e3, 1),
                            "traffic": traffic_for(args.workload, s)}
                   for s, v in stages.items()}
    e.close()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(archive, w, P, args.cpu_budget)
        log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads, "
            f"{cpu['single_thread']['value']} tok/s on 1 ({cpu['sample']})")

    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{w['desc']}, {P}-token prompt + {K} greedy decode steps, fp16 KV cache",
                   "name": args.workload, "prompt_tokens": P, "decode_tokens": K, "batch": 1, "kv_cache": "fp16",
                   "weights": f"seeded N(0,0.02) fp16 quantized (libchpe_pack.so, seed 0)",
                   "parallelism": "none (1 GPU)"},
        "step_roofline": {"bytes_per_step": round(step_bytes), "achieved": round(step_bytes / (wall / K) / 1e9, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(step_bytes / (wall / K) / 1e9 / PEAK_HBM_GBS, 4)},
        "roofline": roofline,
        "stages": stage_table,
        "cpu_baseline": cpu,
        "context_build_s": round(prefill_s, 3),
        "prefill": {"positions": P, "s": round(prefill_s, 3), "tok_s": round(P / prefill_s, 1),
                    "mode": "block steps of 32 tokens" if block else "decode steps"},
        "verify": verify,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
