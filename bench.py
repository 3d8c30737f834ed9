"""Benchmark of the batched ragged decode pass on one MI355X.

    python bench.py [--config c3] [--steps K] [--warmup W] [--gpus 1] [--no-cpu]

Default workload (the metric's configuration): the
27B-class dense q8 model (64 layers, d 5120, 40/8 heads, head_dim 128, FFN
17408, vocab 151936, tied head; random-init int8 weights with one f16 scale
per 32) serving 32 concurrent chats whose contexts are drawn log-uniform in
[128, 16384] (seeded), int8 KV prefilled with random codes. One step = one
packed pass: every chat's next token as one row, 64 blocks with the f16
residual round after each, the LM head and greedy sampling on the GPU; the
sampled ids feed the next step, 128 steps by default (configs[2] decodes 128
tokens per chat). Inputs are resident in HBM when timing starts; each timed
step includes its tiny host->device job table and the device->host copy of
the 32 sampled ids.

The other configurations have lines of their own (`--config c1|c2|c4|c5`),
each one JSON line: c1 the SmolLM2-shaped model (4 chats prefilled, 32 greedy
steps, with the CPU oracle run in full), c2 one 27B block over 12 chats, c4
16 chats x 8 verify rows, c5 the 8B churn (arrivals, 512-token prefill chunks
beside decode rows, retirement). `--hybrid` measures the Qwen3.8-27B hybrid
shape.

Each line carries: `step_roofline`, the whole step's algorithmic bytes per
second against 8 TB/s (the headline fraction); `roofline`, the dominant
kernel's (the q8 matmul for c2-c4, timed with HIP events on the library's
stream); `ceilings`, a read-only stream and a copy measured on the same GPU in
the same process; and `cpu_baseline`, the CPU oracle on the GPU box's host.
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
# HBM bytes per k_gemm_lx launch in configs[2]'s mix, from the FETCH_SIZE and
# WRITE_SIZE counter runs (each calibrated on a plain copy of known size),
# recorded in this summary; the line names it as the traffic's source.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_gemm_lx_c3_traffic.md")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measured_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def _probe():
    path = os.path.join(ROOT, "chattorrent_amd", "libccprobe.so")
    if not os.path.exists(path):
        return None
    lib = C.CDLL(path)
    for name in ("ccp_read_gbps", "ccp_copy_gbps"):
        fn = getattr(lib, name)
        fn.argtypes = [C.c_int, C.c_size_t, C.c_int, C.POINTER(C.c_double)]
        fn.restype = C.c_int
    return lib


def ceilings():
    """The practical HBM ceilings on this GPU, in this process (the probe
    library shares the decode library's HIP runtime): a read-only stream of 8
    GiB, and an 8 GiB device copy (bytes read + written)."""
    lib = _probe()
    if lib is None:
        return None
    out = {}
    for key, fn in (("read_only_GBps", lib.ccp_read_gbps), ("copy_GBps", lib.ccp_copy_gbps)):
        g = C.c_double()
        out[key] = round(g.value, 1) if fn(0, 8 << 30, 5, C.byref(g)) == 0 else None
    return out


def host_info():
    model, mem = None, None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), None)
        with open("/proc/meminfo") as f:
            mem = next((round(int(l.split()[1]) / 1048576, 1) for l in f if l.startswith("MemTotal")), None)
    except OSError:
        pass
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"cpu_model": model, "ram_gib": mem, "host_cpus": os.cpu_count(), "threads": threads}


def copy_calibration(mib):
    """A plain device copy of `mib` MiB, four times (one untimed), for scaling
    the FETCH_SIZE / WRITE_SIZE counters: each copy reads and writes mib MiB."""
    g = C.c_double()
    _probe().ccp_copy_gbps(0, mib << 20, 3, C.byref(g))
    log(f"copied {mib} MiB four times")


def contexts(n, lo, hi, seed):
    from chattorrent_amd import configs
    return configs.workload_contexts(n, lo, hi, seed)


def step_bytes(d, jobs):
    """Algorithmic HBM bytes of one pass: every q8 weight once (int8 + f16
    scale per 32; the LM head only when the pass reaches it), each job's K and
    V rows once per layer (reference layout: 144 B per row at D = 128) for its
    past + n tokens, and its appended rows. jobs: (past, n) pairs."""
    from chattorrent_amd import configs
    kv = configs.kv_token_bytes(d)
    L = d["n_layer"]
    return configs.weight_bytes(d) + sum((p + n) * L * kv + n * L * kv for p, n in jobs)


def step_roofline(bytes_per_step, ms):
    gbs = bytes_per_step / (ms / 1000.0) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": bytes_per_step}


def gemm_roofline(prof, steps, kernel="k_gemm_lx (all q8 projections + LM head)"):
    """The dominant kernel: the q8 matmul (every projection and the LM head),
    its launches timed back-to-back between HIP events on the library's
    stream (cc_profile); achieved = algorithmic bytes / summed launch time."""
    kinds = [k for k in ("qkv", "o", "gate_up", "down", "head") if prof[k][1] > 0]
    g_ms = sum(prof[k][0] for k in kinds)
    g_n = sum(prof[k][1] for k in kinds)
    g_b = sum(prof[k][2] for k in kinds)
    achieved = g_b / (g_ms / 1000.0) / 1e9 if g_ms > 0 else 0.0
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "traffic_source": "profiles/k_gemm_lx_c3_traffic.md: FETCH_SIZE + WRITE_SIZE counter runs of configs[2] "
                              "(each scaled by a plain copy), HBM bytes per launch in that step's mix",
            "kernel": kernel,
            "avg_launch_us": round(g_ms * 1000.0 / max(g_n, 1), 2),
            "bytes_per_launch": round(g_b / max(g_n, 1)),
            "per_kind": {k: {"ms_per_step": round(v[0] / steps, 4), "launches": v[1],
                             "GBps": round(v[2] / (v[0] / 1000.0) / 1e9, 1) if v[0] > 0 else None}
                         for k, v in prof.items()}}


def cpu_oracle_sample(d, jobs, ctxs, seed, layers, reps, head_rows):
    """The CPU oracle (C, OpenMP) on a bounded sample of one pass: `jobs`
    through `layers` distinct blocks (their own weights and KV), `reps` times,
    plus the LM head for `head_rows` rows, scaled to d's depth. Returns (ms per
    full pass, seconds spent)."""
    from oracle import lib as L
    from oracle import model as Mo
    ds = dict(d, n_layer=layers)
    n_max = max(T + j["n"] for T, j in zip(ctxs, jobs)) + 64
    om = Mo.Model(ds, n_slots=len(ctxs), max_pages=-(-n_max // 64))
    om.gen_weights(seed)
    for s, T in enumerate(ctxs):
        if T:
            om.fill_random_kv(s, int(T), seed, s + 1)
    t0 = time.perf_counter()
    for _ in range(reps):
        om.pass_(jobs, head=False)   # rewrites the same new K/V rows each time
    t_blocks = time.perf_counter() - t0
    t_head = 0.0
    if head_rows:
        hs = np.ones((head_rows, d["hidden"]), np.float32)
        t0 = time.perf_counter()
        L.matmul_q8(hs, *om.head_weight(), group=32)
        t_head = time.perf_counter() - t0
    ms = (t_blocks / (layers * reps) * d["n_layer"] + t_head) * 1000.0
    return ms, t_blocks + t_head


def cpu_line(value, unit, sample, kind="port"):
    info = host_info()
    out = {"value": value, "unit": unit, "cores": info["threads"], "kind": kind, "sample": sample}
    out.update(info)
    return out


# The arithmetic: int8 weights (f16 or f32 scales) times f32 activations, the
# activations carried into the MFMAs as two f16 halves, hi + 2^-11 lo (about 22
# significant bits), with f32 products and accumulation.
DTYPE = "int8 x f32 (activations as f16 hi + 2^-11 lo, 22-bit; f32 accumulate)"


def base_line(args, metric, value, unit, ms, dtype=DTYPE):
    return {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype,
            "data": "synthetic: random-init q8 weights (f16 scale per 32), random int8 KV, seeded contexts"}


def profiled(ctx, run, steps):
    """cc_profile over `steps` more passes: each class of each pass relaunched
    back-to-back between one event pair after the pass's own work."""
    ctx.profile(True)
    for _ in range(steps):
        run()
    prof = ctx.profile_read()
    ctx.profile(False)
    return prof


# ------------------------------------------------------------------ c3 ---
def bench_c3(args, ceil):
    """64 layers, 32 chats, greedy decode, one packed pass a step."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    d = dict(configs.M27B)
    chats = args.chats
    pasts = contexts(chats, 128, 16384, args.seed)
    total = args.warmup + args.steps + 16 + args.prof_steps
    n_max = int(64 * math.ceil((pasts.max() + total + 8) / 64))
    log(f"c3: creating context: {d['n_layer']} layers, {chats} chats, n_max {n_max}")
    ctx = Context(d, n_max=n_max, t_max=chats, slots=chats, sessions=chats, max_jobs=chats)
    ctx.fill_random(args.seed)
    for s, T in enumerate(pasts):
        ctx.fill_random_kv(s, int(T), args.seed, s + 1)
    state = {"ids": np.random.default_rng(args.seed + 1).integers(0, d["vocab"], chats), "pasts": pasts}
    ids0, pasts0 = state["ids"].copy(), pasts.copy()
    log(f"c3: contexts {int(pasts.min())}..{int(pasts.max())} mean {pasts.mean():.0f}")

    def step():
        p, toks = state["pasts"], state["ids"]
        jobs = [dict(slot=s, past=int(p[s]), n=1, ids=[int(toks[s])], sampled=1) for s in range(chats)]
        _, out = ctx.step(jobs, topk=1)
        state["ids"] = out[:, 0].astype(np.int64)
        state["pasts"] = p + 1

    slots = list(range(chats))

    def loop(steps):
        """`steps` greedy passes on the device (cc_decode_steps): rows packed
        on the device, each pass fed the previous pass's tokens, one host
        synchronisation at the end."""
        _, out = ctx.decode_steps(slots, state["pasts"], state["ids"], steps, topk=1)
        state["ids"] = out[-1, :, 0].astype(np.int64)
        state["pasts"] = state["pasts"] + steps

    loop(args.warmup)
    timed = [state["pasts"] + k for k in range(args.steps)]
    t0 = time.perf_counter()
    loop(args.steps)
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    # the same passes driven one cc_step at a time from the host, for comparison
    host_steps = 16
    t0 = time.perf_counter()
    for _ in range(host_steps):
        step()
    host_ms = (time.perf_counter() - t0) * 1000.0 / host_steps
    tok_s = chats / (ms / 1000.0)
    bytes_avg = float(np.mean([step_bytes(d, [(int(p), 1) for p in ps]) for ps in timed]))
    sr = step_roofline(bytes_avg, ms)
    log(f"c3: {ms:.3f} ms/step, {tok_s:.1f} tok/s, {bytes_avg / 1e9:.2f} GB/step -> {sr['achieved']:.0f} GB/s "
        f"({sr['frac'] * 100:.1f}% of 8 TB/s); one cc_step at a time: {host_ms:.3f} ms/step")
    roof = gemm_roofline(profiled(ctx, step, args.prof_steps), args.prof_steps)
    ctx.close()
    log(f"c3: profile {json.dumps(roof['per_kind'])}")
    cpu = None
    if not args.no_cpu:
        log("c3: timing the CPU oracle sample")
        jobs = [dict(slot=s, past=int(T), n=1, ids=[int(ids0[s])], sampled=1, topk=1) for s, T in enumerate(pasts0)]
        ms_cpu, secs = cpu_oracle_sample(d, jobs, [int(T) for T in pasts0], args.seed, args.cpu_layers,
                                         args.cpu_reps, chats)
        cpu = cpu_line(round(chats / (ms_cpu / 1000.0), 3), "tok/s",
                       f"oracle (C restatement, OpenMP): the 32-row decode pass through {args.cpu_layers} distinct "
                       f"27B blocks timed {args.cpu_reps} times plus the LM head for 32 rows ({secs:.1f} s), scaled "
                       f"to 64 blocks ({ms_cpu:.0f} ms/step)")
    line = base_line(args, "aggregate decode tok/s @32 ragged chats, 27B q8; % of HBM roofline", tok_s, "tok/s", ms)
    line["config"] = {"workload": "configs[2]: 27B-class q8 (64 layers, d5120, 40/8 heads, ffn 17408, vocab 151936), "
                                  "32 chats, contexts log-uniform [128,16384], greedy decode, one packed pass per step",
                      "chats": chats, "layers": d["n_layer"], "mean_context": float(pasts0.mean()),
                      "step_hbm_bytes": bytes_avg, "step_frac_of_hbm_peak": sr["frac"],
                      "timed_loop": "cc_decode_steps: all timed passes enqueued back to back, packed on the device",
                      "host_loop_ms_per_step": round(host_ms, 4)}
    line["step_roofline"] = sr
    line["roofline"] = roof
    line["ceilings"] = ceil
    if ceil and ceil.get("read_only_GBps"):
        sr["frac_of_read_only"] = round(sr["achieved"] / ceil["read_only_GBps"], 4)
    line["cpu_baseline"] = cpu
    return line


# ------------------------------------------------------------------ c2 ---
def bench_c2(args, ceil):
    """one 27B-class block, 12 chats with contexts U[256, 16384],
    one decode row each entering as f16 ~N(0, 1) rows."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    from oracle import lib as L
    from oracle import model as Mo
    d = dict(configs.BLOCK27B)
    rng = np.random.default_rng(args.seed)
    pasts = [int(t) for t in rng.integers(256, 16385, 12)]
    ctx = Context(d, n_max=16384 + 64 * 4, t_max=16, slots=12, sessions=12, max_jobs=12)
    ctx.fill_random(args.seed)
    for s, T in enumerate(pasts):
        ctx.fill_random_kv(s, T, args.seed, s + 1)
    entry = L.to_f16(rng.standard_normal((12, d["hidden"])).astype(np.float32))
    jobs = [dict(slot=s, past=T, n=1, hidden=entry[s:s + 1]) for s, T in enumerate(pasts)]
    run = lambda: ctx.step(jobs, at=1, to=2)
    for _ in range(args.warmup):
        run()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    roof = gemm_roofline(profiled(ctx, run, args.prof_steps), args.prof_steps)
    ctx.close()
    # one block: its weights (no embedding or head) and the chats' K/V rows
    from chattorrent_amd import configs as Cf
    b = Cf.weight_bytes(dict(d, vocab=0)) + sum((T + 1) * Cf.kv_token_bytes(d) + Cf.kv_token_bytes(d) for T in pasts)
    cpu = None
    if not args.no_cpu:
        om = Mo.Model(d, n_slots=12, max_pages=16384 // 64 + 4)
        om.gen_weights(args.seed)
        for s, T in enumerate(pasts):
            om.fill_random_kv(s, T, args.seed, s + 1)
        oj = [dict(j, hidden=L.from_f16(j["hidden"])) for j in jobs]
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            om.pass_(oj, head=False)
        ms_cpu = (time.perf_counter() - t0) * 1000.0 / reps
        cpu = cpu_line(round(1000.0 / ms_cpu, 3), "block passes/s",
                       f"oracle (C restatement, OpenMP): the whole 12-chat block pass, {reps} times "
                       f"({ms_cpu:.0f} ms each)")
    line = base_line(args, "one 27B-class block pass over 12 ragged chats (block passes/s); % of HBM roofline",
                     1000.0 / ms, "block passes/s", ms)
    line["config"] = {"workload": "configs[1]: one 27B-class block (d5120, 40/8 heads, D128, ffn 17408), 12 chats, "
                                  "contexts U[256,16384], one f16 ~N(0,1) row each",
                      "mean_context": float(np.mean(pasts))}
    line["step_roofline"] = step_roofline(b, ms)
    line["roofline"] = roof
    line["ceilings"] = ceil
    line["cpu_baseline"] = cpu
    return line


# ------------------------------------------------------------------ c4 ---
def bench_c4(args, ceil):
    """16 chats x 8 verify rows (1 real + 7 random drafts) on the
    full 27B-class model, contexts U[4096, 32768], every row sampled and the
    drafts accepted by per-row argmax."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    d = dict(configs.M27B)
    rng = np.random.default_rng(args.seed + 3)
    chats, n = 16, 8
    pasts0 = np.array([int(t) for t in rng.integers(4096, 32769, chats)])
    total = args.warmup + args.steps + args.prof_steps
    n_max = int(64 * math.ceil((pasts0.max() + n * total + 8) / 64))
    log(f"c4: creating context, n_max {n_max}")
    ctx = Context(d, n_max=n_max, t_max=chats * n, slots=chats, sessions=chats, max_jobs=chats)
    ctx.fill_random(args.seed)
    for s, T in enumerate(pasts0):
        ctx.fill_random_kv(s, int(T), args.seed, s + 1)
    state = {"pasts": pasts0.copy(), "accepted": 0}

    def step():
        p = state["pasts"]
        drafts = rng.integers(0, d["vocab"], (chats, n))
        jobs = [dict(slot=s, past=int(p[s]), n=n, ids=[int(x) for x in drafts[s]], sampled=n) for s in range(chats)]
        _, ids = ctx.step(jobs, topk=1)
        got = ids[:, 0].reshape(chats, n)
        for s in range(chats):
            a = 0
            while a < n - 1 and got[s, a] == drafts[s, a + 1]:
                a += 1
            state["accepted"] += a
        state["pasts"] = p + n

    for _ in range(args.warmup):
        step()
    timed = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        timed.append(state["pasts"].copy())
        step()
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    roof = gemm_roofline(profiled(ctx, step, args.prof_steps), args.prof_steps,
                         kernel="k_gemm_tm (all q8 projections at 128 rows; the LM head too)")
    ctx.close()
    b = float(np.mean([step_bytes(d, [(int(p), n) for p in ps]) for ps in timed]))
    line = base_line(args, "speculative verify rows/s, 16 chats x 8 rows, 27B q8; % of HBM roofline",
                     chats * n / (ms / 1000.0), "rows/s", ms)
    line["config"] = {"workload": "configs[3]: 27B-class q8, 16 chats x 8 verify rows (1 real + 7 random drafts), "
                                  "contexts U[4096,32768], causal within each run, per-row argmax acceptance",
                      "mean_context": float(np.mean([ps.mean() for ps in timed])),
                      "drafts_accepted": state["accepted"]}
    line["step_roofline"] = step_roofline(b, ms)
    line["roofline"] = roof
    line["ceilings"] = ceil
    cpu = None
    if not args.no_cpu:
        log("c4: timing the CPU oracle sample")
        jobs = [dict(slot=s, past=int(T), n=n, ids=[1] * n, sampled=n, topk=1) for s, T in enumerate(pasts0)]
        ms_cpu, secs = cpu_oracle_sample(d, jobs, [int(T) for T in pasts0], args.seed, 2, 1, chats * n)
        cpu = cpu_line(round(chats * n / (ms_cpu / 1000.0), 3), "rows/s",
                       f"oracle (C restatement, OpenMP): the 128-row verify pass through 2 distinct 27B blocks plus "
                       f"the LM head for 128 rows ({secs:.1f} s), scaled to 64 blocks ({ms_cpu:.0f} ms/pass)")
    line["cpu_baseline"] = cpu
    return line


# ------------------------------------------------------------------ c5 ---
def bench_c5(args, ceil):
    """continuous batching on the 8B shape: 64 chat slots,
    Poisson(2) arrivals a step, prompts log-uniform in [32, 4096] fed as
    512-token chunks beside the decode rows in one pass, chats retiring after
    U[64, 512] generated tokens. The pass is MFMA-bound once its rows pass
    about 150: the line reports tokens processed per second and the matmul
    FLOP rate against the dense f16 MFMA peak."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    d = dict(configs.LLAMA8B)
    slots, chunk, t_max = 64, 512, 64 + 2 * 512
    n_max = 4096 + 512 + 64
    ctx = Context(d, n_max=n_max, t_max=t_max, slots=slots, sessions=slots, max_jobs=slots)
    ctx.fill_random(args.seed)
    churn = configs.Churn(d["vocab"], slots, chunk, t_max, args.seed + 5)

    def one_step():
        jobs = churn.jobs()
        if not jobs:
            return
        _, ids = ctx.step(jobs, topk=1)
        for f in churn.advance(jobs, ids[:, 0]):
            ctx.release(f)

    for _ in range(args.warmup):
        one_step()
    stats = churn.stats
    for k in stats:
        stats[k] = 0
    t0 = time.perf_counter()
    for k in range(args.steps):
        one_step()
        if k % 250 == 249:
            log(f"c5: {k + 1} steps, {len(churn.chats)} chats")
    secs = time.perf_counter() - t0
    prof = profiled(ctx, one_step, args.prof_steps)
    ctx.close()
    ms = secs * 1000.0 / args.steps
    params = configs.weight_bytes(d) / (1 + 2 / 32)
    tflops = 2.0 * stats["rows"] * params / secs / 1e12
    line = base_line(args, "continuous-batching tokens processed/s (prefill + decode), 8B q8, 64 slots",
                     stats["rows"] / secs, "tok/s", ms)
    line["config"] = {"workload": "configs[4]: Llama-3.1-8B-shaped q8, 64 slots, Poisson(2) arrivals/step, prompts "
                                  "log-uniform [32,4096] in 512-token chunks beside decode rows, retire at U[64,512]",
                      "decode_tok_s": round(stats["decode"] / secs, 2),
                      "prefill_tok_s": round(stats["prefill"] / secs, 2),
                      "rows_per_step": round(stats["rows"] / args.steps, 1), "arrived": stats["arrived"],
                      "retired": stats["retired"],
                      "per_kind_ms_per_step": {k: round(v[0] / args.prof_steps, 4) for k, v in prof.items()}}
    line["roofline"] = {"bound": "mfma", "achieved": round(tflops, 1), "peak": F16_MFMA_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / F16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                        "note": "algorithmic FLOPs 2 x rows x params per pass; the matmul issues each product twice "
                                "(f16 hi and lo halves of the f32 activations)"}
    line["ceilings"] = ceil
    line["cpu_baseline"] = None
    if not args.no_cpu:
        log("c5: timing the CPU oracle sample")
        ms_cpu, rows, secs = cpu_churn_sample(d, slots, chunk, t_max, args.seed, passes=3)
        line["cpu_baseline"] = cpu_line(
            round(rows / (ms_cpu / 1000.0), 3), "tok/s",
            f"oracle (C restatement, OpenMP): the churn's first 3 passes ({rows} rows, prompt chunks and decode "
            f"rows) through one 8B block ({secs:.1f} s) plus the LM head for their sampled rows, scaled to 32 "
            f"blocks ({ms_cpu:.0f} ms for the 3 passes)")
    return line


def cpu_churn_sample(d, slots, chunk, t_max, seed, passes):
    """The CPU oracle on configs[4]'s first `passes` passes (the same Churn
    workload, seeded alike): every pass's rows through one block with its own
    weights, and the LM head for the pass's sampled rows, scaled to d's depth.
    Returns (ms for the passes at full depth, rows, seconds spent)."""
    from chattorrent_amd import configs
    from oracle import lib as L
    from oracle import model as Mo
    ds = dict(d, n_layer=1)
    n_max = 4096 + 512 + 64
    om = Mo.Model(ds, n_slots=slots, max_pages=-(-n_max // 64))
    om.gen_weights(seed)
    churn = configs.Churn(d["vocab"], slots, chunk, t_max, seed + 5)
    t_blocks = t_head = 0.0
    rows = 0
    for _ in range(passes):
        jobs = churn.jobs()
        t0 = time.perf_counter()
        om.pass_(jobs, head=False)
        t_blocks += time.perf_counter() - t0
        sampled = sum(j["sampled"] for j in jobs)
        if sampled:
            hs = np.ones((sampled, d["hidden"]), np.float32)
            t0 = time.perf_counter()
            L.matmul_q8(hs, *om.head_weight(), group=32)
            t_head += time.perf_counter() - t0
        rows += sum(j["n"] for j in jobs)
        churn.advance(jobs, np.zeros(sampled, np.int64))
    return (t_blocks * d["n_layer"] + t_head) * 1000.0, rows, t_blocks + t_head


def js_sample(d, lens, prompts, seed, steps=3):
    """The "JS path" analogue: the single-threaded JavaScript restatement of
    the pass (oracle/js/decode.js) on configs[0]'s model, decoding `steps`
    greedy passes of the 4 chats at contexts `lens` over generated K/V rows
    (the same shapes as after the prefill). None when node is absent."""
    import shutil
    import tempfile
    from oracle import jsdecode as J
    if J.node_binary() is None:
        return None
    path = tempfile.mkdtemp(prefix="ccjs-")
    try:
        t0 = time.perf_counter()
        J.write_inputs(path, d, seed, lens, [int(p[-1]) for p in prompts], steps)
        log(f"c1: JS inputs written in {time.perf_counter() - t0:.1f} s; running {steps} single-thread JS passes")
        r = J.run(path, steps)
    finally:
        shutil.rmtree(path, ignore_errors=True)
    return {"value": round(4 / (r["ms_per_step"] / 1000.0), 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"oracle/js/decode.js (Node, one thread): {steps} greedy passes of the 4 chats at contexts "
                      f"{list(lens)} ({r['ms_per_step']:.0f} ms/pass)"}


# ------------------------------------------------------------------ c1 ---
def bench_c1(args, ceil):
    """the SmolLM2-shaped model (30 layers), 4 chats whose prompts
    of {17, 130, 511, 1024} random ids are prefilled in one pass, then 32
    greedy steps of one 4-row pass each (timed); the CPU oracle runs the same
    decode in full."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    from oracle import lib as L
    from oracle import model as Mo
    d = dict(configs.SMOLLM2)
    lens = [17, 130, 511, 1024]
    steps = 32
    n_max = 64 * math.ceil((max(lens) + steps + 1) / 64)
    prompts = [L.gen_ids(args.seed, 0x5EED + s, n, d["vocab"]) for s, n in enumerate(lens)]

    def run_gpu():
        ctx = Context(d, n_max=n_max, t_max=sum(lens), slots=4)
        ctx.fill_random(args.seed)
        _, ids = ctx.step([dict(slot=s, past=0, n=n, ids=prompts[s], sampled=1) for s, n in enumerate(lens)])
        toks = ids[:, 0].astype(np.int64)
        t0 = time.perf_counter()
        for k in range(steps):
            _, ids = ctx.step([dict(slot=s, past=lens[s] + k, n=1, ids=[int(toks[s])], sampled=1) for s in range(4)])
            toks = ids[:, 0].astype(np.int64)
        ms = (time.perf_counter() - t0) * 1000.0 / steps
        ctx.close()
        return ms

    for _ in range(args.warmup):
        run_gpu()
    ms = run_gpu()
    b = float(np.mean([step_bytes(d, [(lens[s] + k, 1) for s in range(4)]) for k in range(steps)]))
    cpu = None
    if not args.no_cpu:
        om = Mo.Model(d, n_slots=4, max_pages=n_max // 64)
        om.gen_weights(args.seed)
        out = om.pass_([dict(slot=s, past=0, n=n, ids=prompts[s], sampled=1, topk=1) for s, n in enumerate(lens)])
        toks = [int(o["ids"][0][0]) for o in out]
        t0 = time.perf_counter()
        for k in range(steps):
            out = om.pass_([dict(slot=s, past=lens[s] + k, n=1, ids=[toks[s]], sampled=1, topk=1) for s in range(4)])
            toks = [int(o["ids"][0][0]) for o in out]
        ms_cpu = (time.perf_counter() - t0) * 1000.0 / steps
        cpu = cpu_line(round(4 / (ms_cpu / 1000.0), 3), "tok/s",
                       f"oracle (C restatement, OpenMP): all 32 decode steps of the 4 chats after its own prefill "
                       f"({ms_cpu:.1f} ms/step)")
        cpu["js_single_thread"] = js_sample(d, lens, prompts, args.seed)
    line = base_line(args, "aggregate decode tok/s @4 ragged chats, SmolLM2-135M-shaped q8", 4 / (ms / 1000.0),
                     "tok/s", ms)
    line["steps"] = steps
    line["config"] = {"workload": "configs[0]: SmolLM2-135M-shaped q8 (30 layers, d576, 9/3 heads, ffn 1536, vocab "
                                  "49152), 4 chats prefilled {17,130,511,1024}, 32 greedy steps of one 4-row pass"}
    line["step_roofline"] = step_roofline(b, ms)
    line["ceilings"] = ceil
    line["cpu_baseline"] = cpu
    return line


# -------------------------------------------------------------- hybrid ---
def bench_hybrid(args, ceil):
    """Decode over the Qwen3.8-27B hybrid shape (48 Gated DeltaNet + 16
    full-attention blocks, untied 248320-row head): the same ragged 32-chat
    step as the headline, on synthetic weights (the linear blocks' f32
    parameters fixed), then the MTP head's 7-draft chain for one session."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    d = dict(configs.QWEN38)
    chats = args.chats
    pasts = contexts(chats, 128, 16384, args.seed)
    total = args.warmup + args.steps + 2
    n_max = int(64 * math.ceil((pasts.max() + total + 16) / 64))
    log(f"hybrid: creating context, {chats} chats, n_max {n_max}")
    ctx = Context(d, n_max=n_max, t_max=chats, slots=chats, sessions=chats, max_jobs=chats)
    ctx.fill_random(args.seed)
    for s, T in enumerate(pasts):
        ctx.fill_random_kv(s, int(T), args.seed, s + 1)
    state = {"ids": np.random.default_rng(args.seed + 1).integers(0, 65536, chats), "pasts": pasts}

    def step():
        p, toks = state["pasts"], state["ids"]
        jobs = [dict(slot=s, past=int(p[s]), n=1, ids=[int(toks[s]) % 65536], sampled=1) for s in range(chats)]
        _, out = ctx.step(jobs, topk=1)
        state["ids"] = out[:, 0].astype(np.int64)
        state["pasts"] = p + 1

    for _ in range(args.warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    prof = profiled(ctx, step, 1)
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        ctx.mtp_draft(0, 0, int(state["ids"][0]) % 65536, int(state["pasts"][0]), 7)
    mtp_ms = (time.perf_counter() - t0) * 1000.0 / reps
    st = ctx.stats()
    ctx.close()
    line = base_line(args, "hybrid decode tok/s @32 ragged chats, Qwen3.8-27B shape (48 Gated DeltaNet + 16 "
                           "full-attention blocks), q8", chats / (ms / 1000.0), "tok/s", ms)
    line["data"] = "synthetic: random-init q8 weights, fixed Gated DeltaNet parameters, random int8 KV"
    line["mtp_chain_7_drafts_ms"] = round(mtp_ms, 3)
    line["per_kind_ms_per_step"] = {k: round(v[0], 4) for k, v in prof.items()}
    line["vram_gb"] = round(st["vram_bytes"] / 1e9, 2)
    line["config"] = {"workload": "Qwen3.8-27B shape, 32 chats, contexts log-uniform [128,16384]",
                      "mean_context": float(pasts.mean())}
    line["ceilings"] = ceil
    return line


CONFIGS = {"c1": bench_c1, "c2": bench_c2, "c3": bench_c3, "c4": bench_c4, "c5": bench_c5}
DEFAULT_STEPS = {"c1": 32, "c2": 50, "c3": 128, "c4": 10, "c5": 2000}   # c5: configs[4]'s 2000 steps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prof-steps", type=int, default=8, help="passes of the per-kernel profile replay")
    ap.add_argument("--chats", type=int, default=32)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=8)
    ap.add_argument("--cpu-reps", type=int, default=7)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (for scaling the HBM byte counters) and exit")
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
    if args.steps is None:
        args.steps = DEFAULT_STEPS["c3" if args.hybrid else args.config]
    ceil = ceilings()
    log(f"ceilings {ceil}")
    line = bench_hybrid(args, ceil) if args.hybrid else CONFIGS[args.config](args, ceil)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
