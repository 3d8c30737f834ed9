"""Benchmark of the batched ragged decode pass on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config c3] [--no-cpu]

Workload (the metric's configuration): the
27B-class dense q8 model (64 layers, d 5120, 40/8 heads, head_dim 128, FFN
17408, vocab 151936, tied head; random-init int8 weights with one f16 scale
per 32) serving 32 concurrent chats whose contexts are drawn log-uniform in
[128, 16384] (seeded), int8 KV prefilled with random codes. One step = one
packed pass: every chat's next token as one row, 64 blocks with the f16
residual round after each, the LM head and greedy sampling on the GPU; the
sampled ids feed the next step. Inputs are resident in HBM when timing
starts; each timed step includes its tiny host->device job table and the
device->host copy of the 32 sampled ids.

Prints one JSON line: aggregate decode tok/s, the HBM roofline of the
dominant kernel (the q8 projection GEMM, timed with HIP events on the
library's stream; also against a measured device-copy bandwidth), and the
CPU oracle timed on a bounded sample of the same step.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per k_gemm_lx launch, from the FETCH_SIZE and WRITE_SIZE counter
# runs (each calibrated on a plain copy of known size); written by hand into
# this summary after those runs, read here so the JSON line carries it.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemm_lx_c3_traffic.md")


def measured_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def copy_calibration(mib):
    """A plain device-to-device copy of `mib` MiB, three times, for scaling
    the FETCH_SIZE / WRITE_SIZE counters: each copy reads and writes exactly
    mib MiB."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"[bench] copied {mib} MiB three times", file=sys.stderr, flush=True)


def contexts(n, lo, hi, seed):
    from chattorrent_amd import configs
    return configs.workload_contexts(n, lo, hi, seed)


def step_bytes(d, pasts):
    """Algorithmic HBM bytes of one decode step: every q8 weight once (int8 +
    f16 scale per 32), every chat's K and V rows once per layer (reference
    layout: 144 B per row at D = 128), and the appended rows."""
    from chattorrent_amd import configs
    kv = configs.kv_token_bytes(d)
    L = d["n_layer"]
    return configs.weight_bytes(d) + sum(int(p) + 1 for p in pasts) * L * kv + len(pasts) * L * kv


def cpu_baseline(d, pasts, ids, seed, layers=8, reps=7):
    """The CPU oracle (C, OpenMP) on a bounded sample of the same step: the
    32-row pass through `layers` distinct blocks (their own weights and KV),
    timed `reps` times over (about 10 s of CPU work on a 16-thread host), plus
    the LM head for all 32 rows, scaled to the 64-block step."""
    from oracle import model as Mo
    from oracle import lib as L
    import oracle.lib  # noqa: F401
    ds = dict(d, n_layer=layers)
    n_max = int(max(pasts)) + 2
    om = Mo.Model(ds, n_slots=len(pasts), max_pages=-(-n_max // 64))
    om.gen_weights(seed)
    for s, T in enumerate(pasts):
        om.fill_random_kv(s, int(T), seed, s + 1)
    jobs = [dict(slot=s, past=int(T), n=1, ids=[int(ids[s])], sampled=1, topk=1) for s, T in enumerate(pasts)]
    t0 = time.perf_counter()
    for _ in range(reps):
        om.pass_(jobs, head=False)   # rewrites the same new K/V rows each time
    t_blocks = time.perf_counter() - t0
    hs = np.ones((len(pasts), d["hidden"]), np.float32)
    t0 = time.perf_counter()
    L.matmul_q8(hs, *om.head_weight(), group=32)
    t_head = time.perf_counter() - t0
    per_block = t_blocks / (layers * reps)
    ms_step = (per_block * d["n_layer"] + t_head) * 1000.0
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(len(pasts) / (ms_step / 1000.0), 3), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle (C restatement, OpenMP, {threads} threads): the 32-row decode pass through {layers} "
                      f"distinct 27B blocks timed {reps} times ({layers * reps} block passes, {t_blocks:.1f} s) "
                      f"plus the LM head ({t_head:.2f} s), scaled to 64 blocks ({ms_step:.0f} ms/step)"}


def stream_copy_gbs(gib=2, iters=5):
    """Device-to-device copy bandwidth (bytes read + written per second) of a
    plain copy of `gib` GiB, the practical ceiling the pass is also compared
    against; torch's copy on torch's stream, timed with its events. Runs in a
    child process of its own (--stream-copy): torch carries its own HIP
    runtime, which cannot share a process with the library's."""
    import torch
    n = gib << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        b.copy_(a)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / iters
    del a, b
    torch.cuda.empty_cache()
    return 2.0 * n / (ms / 1000.0) / 1e9


def hybrid_main(args):
    """Decode over the Qwen3.8-27B hybrid shape (48 Gated DeltaNet + 16
    full-attention blocks, untied 248320-row head): the same ragged 32-chat
    step as the headline, on synthetic weights (the linear blocks' f32
    parameters fixed), then the MTP head's 7-draft chain for one session."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    d = dict(configs.QWEN38)
    chats = args.chats
    pasts = contexts(chats, 128, 16384, args.seed)
    total = args.warmup + args.steps
    n_max = int(64 * math.ceil((pasts.max() + total + 16) / 64))
    print(f"[bench] hybrid: creating context, {chats} chats, n_max {n_max}", file=sys.stderr, flush=True)
    ctx = Context(d, n_max=n_max, t_max=chats, slots=chats, sessions=chats, max_jobs=chats)
    ctx.fill_random(args.seed)
    for s, T in enumerate(pasts):
        ctx.fill_random_kv(s, int(T), args.seed, s + 1)
    ids = np.random.default_rng(args.seed + 1).integers(0, 65536, chats)

    def step(p, toks):
        jobs = [dict(slot=s, past=int(p[s]), n=1, ids=[int(toks[s]) % 65536], sampled=1) for s in range(chats)]
        _, out = ctx.step(jobs, topk=1)
        return out[:, 0].astype(np.int64)

    for _ in range(args.warmup):
        ids = step(pasts, ids)
        pasts = pasts + 1
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ids = step(pasts, ids)
        pasts = pasts + 1
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    ctx.profile(True)
    ids = step(pasts, ids)
    pasts = pasts + 1
    prof = ctx.profile_read()
    ctx.profile(False)
    # the MTP chain after the last row of session 0 (cc_mtp_draft, 7 drafts)
    t0 = time.perf_counter()
    reps = 10
    for r in range(reps):
        ctx.mtp_draft(0, 0, int(ids[0]) % 65536, int(pasts[0]), 7)
    mtp_ms = (time.perf_counter() - t0) * 1000.0 / reps
    st = ctx.stats()
    line = {"metric": "hybrid decode tok/s @32 ragged chats, Qwen3.8-27B shape (48 Gated DeltaNet + 16 "
                      "full-attention blocks), q8", "value": round(chats / (ms / 1000.0), 2), "unit": "tok/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "dtype": "int8xf32",
            "data": "synthetic: random-init q8 weights, fixed Gated DeltaNet parameters, random int8 KV",
            "mtp_chain_7_drafts_ms": round(mtp_ms, 3),
            "per_kind_ms_per_step": {k: round(v[0], 4) for k, v in prof.items()},
            "vram_gb": round(st["vram_bytes"] / 1e9, 2),
            "config": {"workload": "Qwen3.8-27B shape, 32 chats, contexts log-uniform [128,16384]",
                       "mean_context": float(pasts.mean())}}
    print(json.dumps(line), flush=True)
    ctx.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--chats", type=int, default=32)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=8)
    ap.add_argument("--cpu-reps", type=int, default=7)
    ap.add_argument("--layers", type=int, default=None, help="fewer layers (debug only; not a valid bench)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (for scaling the HBM byte counters) and exit")
    ap.add_argument("--stream-copy", action="store_true", help="only print the device copy bandwidth and exit")
    ap.add_argument("--hybrid", action="store_true",
                    help="the Qwen3.8-27B hybrid shape instead (its own line; not the headline metric)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: every box here has one GPU and this build has no multi-GPU path "
              "(the pass would scale as one data-parallel replica per GPU, with no exchange).", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.stream_copy:
        print(f"STREAM_COPY_GBPS {stream_copy_gbs():.3f}", flush=True)
        return
    if args.hybrid:
        hybrid_main(args)
        return
    # before this process touches the GPU: the copy ceiling, from a child process
    import subprocess
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--stream-copy"], capture_output=True, text=True,
                       timeout=600)
    copy_gbs = None
    for line in r.stdout.splitlines():
        if line.startswith("STREAM_COPY_GBPS"):
            copy_gbs = float(line.split()[1])
    if copy_gbs is None:
        print(f"[bench] stream copy measurement failed (rc {r.returncode}): {r.stderr[-400:]}", file=sys.stderr)
    else:
        print(f"[bench] stream copy {copy_gbs:.0f} GB/s", file=sys.stderr, flush=True)

    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context

    d = dict(configs.M27B)
    if args.layers:
        d["n_layer"] = args.layers
    chats = args.chats
    pasts = contexts(chats, 128, 16384, args.seed)
    total = args.warmup + args.steps
    n_max = int(64 * math.ceil((pasts.max() + total + 8) / 64))
    print(f"[bench] creating context: {d['n_layer']} layers, {chats} chats, n_max {n_max}", file=sys.stderr,
          flush=True)
    ctx = Context(d, n_max=n_max, t_max=chats, slots=chats, sessions=chats, max_jobs=chats)
    ctx.fill_random(args.seed)
    for s, T in enumerate(pasts):
        ctx.fill_random_kv(s, int(T), args.seed, s + 1)
    ids = np.random.default_rng(args.seed + 1).integers(0, d["vocab"], chats)
    ids0 = ids.copy()
    pasts0 = pasts.copy()
    print(f"[bench] filled weights and KV; contexts {int(pasts.min())}..{int(pasts.max())} "
          f"mean {pasts.mean():.0f}", file=sys.stderr, flush=True)

    def step(p, toks):
        jobs = [dict(slot=s, past=int(p[s]), n=1, ids=[int(toks[s])], sampled=1) for s in range(chats)]
        _, out = ctx.step(jobs, topk=1)
        return out[:, 0].astype(np.int64)

    for _ in range(args.warmup):
        ids = step(pasts, ids)
        pasts = pasts + 1
    timed_pasts = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        timed_pasts.append(pasts.copy())
        ids = step(pasts, ids)
        pasts = pasts + 1
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    tok_s = chats / (ms / 1000.0)
    bytes_avg = float(np.mean([step_bytes(d, p) for p in timed_pasts]))
    step_frac = bytes_avg / (ms / 1000.0) / (HBM_PEAK_GBS * 1e9)
    print(f"[bench] {ms:.3f} ms/step, {tok_s:.1f} tok/s, step bytes {bytes_avg / 1e9:.2f} GB "
          f"-> {bytes_avg / (ms / 1000.0) / 1e9:.0f} GB/s ({step_frac * 100:.1f}% of 8 TB/s)",
          file=sys.stderr, flush=True)

    # The dominant kernel: the q8 projection GEMM (every block's q|k|v, o,
    # gate|up and down, and the LM head), timed with HIP events on the
    # library's stream over a second region of the same steps: in profile
    # mode each step relaunches each class for all 64 blocks back-to-back
    # between one event pair (a marker beside every launch would add a few
    # microseconds of gap to each), so ms / launches is a launch's duration.
    ctx.profile(True)
    for _ in range(args.steps):
        ids = step(pasts, ids)
        pasts = pasts + 1
    prof = ctx.profile_read()
    ctx.profile(False)
    g_ms = sum(prof[k][0] for k in ("qkv", "o", "gate_up", "down", "head"))
    g_n = sum(prof[k][1] for k in ("qkv", "o", "gate_up", "down", "head"))
    g_b = sum(prof[k][2] for k in ("qkv", "o", "gate_up", "down", "head"))
    achieved = g_b / (g_ms / 1000.0) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "kernel": "k_gemm_lx (all q8 projections + LM head)",
            "avg_launch_us": round(g_ms * 1000.0 / max(g_n, 1), 2),
            "bytes_per_launch": round(g_b / max(g_n, 1)),
            "per_kind": {k: {"ms_per_step": round(v[0] / args.steps, 4), "launches": v[1],
                             "GBps": round(v[2] / (v[0] / 1000.0) / 1e9, 1) if v[0] > 0 else None}
                         for k, v in prof.items()}}
    print(f"[bench] profile: {json.dumps(roof['per_kind'])}", file=sys.stderr, flush=True)
    # the practical ceiling beside the nominal 8 TB/s: a plain device copy
    roof["stream_copy_GBps"] = round(copy_gbs, 1) if copy_gbs else None
    roof["frac_of_stream_copy"] = round(achieved / copy_gbs, 4) if copy_gbs else None
    cpu = None
    if not args.no_cpu:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        cpu = cpu_baseline(d, pasts0, ids0, args.seed, layers=args.cpu_layers, reps=args.cpu_reps)
    line = {
        "metric": "aggregate decode tok/s @32 ragged chats, 27B q8; % of HBM roofline",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8xf32",
        "data": "synthetic: random-init q8 weights, random int8 KV, seeded contexts",
        "config": {"workload": "configs[2]: 27B-class q8 (64 layers, d5120, 40/8 heads, ffn 17408, vocab 151936), "
                               "32 chats, contexts log-uniform [128,16384], greedy decode, one packed pass per step",
                   "chats": chats, "layers": d["n_layer"], "mean_context": float(pasts0.mean()),
                   "step_hbm_bytes": bytes_avg, "step_frac_of_hbm_peak": round(step_frac, 4),
                   "step_frac_of_stream_copy": round(bytes_avg / (ms / 1000.0) / 1e9 / copy_gbs, 4) if copy_gbs
                   else None},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    ctx.close()


if __name__ == "__main__":
    main()
