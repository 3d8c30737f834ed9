"""Model shapes of the benchmark configurations (dims as loader.js
dimsFromManifest names them, web/model/loader.js:146-201).

The shapes are the ones the benchmark names; RoPE theta and eps are not given
there and are pinned here. SmolLM2's come from the reference's DIMS
(web/model/kernels.js:23-37); the 27B-class and 8B shapes use theta 1e6 /
eps 1e-6 and Llama 3.1's published values respectively.
"""

SMOLLM2 = dict(hidden=576, n_layer=30, n_heads=9, n_kv_heads=3, head_dim=64, ffn=1536, vocab=49152,
               rms_eps=1e-5, rope_theta=100000.0, tied=True, group_q8=32)

# 27B-class dense block: d 5120, 40 q / 8 kv heads, head_dim 128, SwiGLU 17408.
M27B = dict(hidden=5120, n_layer=64, n_heads=40, n_kv_heads=8, head_dim=128, ffn=17408, vocab=151936,
            rms_eps=1e-6, rope_theta=1000000.0, tied=True, group_q8=32)

BLOCK27B = dict(M27B, n_layer=1)

LLAMA8B = dict(hidden=4096, n_layer=32, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
               rms_eps=1e-5, rope_theta=500000.0, tied=False, group_q8=32,
               rope_scaling=dict(factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                                 original_max_position_embeddings=8192))


def with_layers(d, n):
    out = dict(d)
    out["n_layer"] = n
    return out


def weight_bytes(d):
    """Stored bytes of the q8 weights: int8 + one f16 scale per 32 (1.0625 B/w),
    embedding counted once when tied (web/model/model.js:721-734 weightBudget)."""
    H, D, F = d["hidden"], d["head_dim"], d["ffn"]
    per_layer = (d["n_heads"] * D * H + 2 * d["n_kv_heads"] * D * H + H * d["n_heads"] * D + 3 * F * H)
    params = d["n_layer"] * per_layer + d["vocab"] * H * (1 if d.get("tied", True) else 2)
    return params * (1 + 2 / 32)


def kv_token_bytes(d):
    """K and V bytes of one token in one layer: web/split.js:132 kvRowBytes x 2."""
    D = d["head_dim"]
    return 2 * d["n_kv_heads"] * (D + 4 * D // min(32, D))

# Qwen3.8-27B (the reference's shipped hybrid, web/model/model.js:411-576):
# 48 Gated DeltaNet blocks and 16 full-attention blocks (three to one), the
# full ones with 24 query / 4 kv heads of 256 (a quarter rotary), the linear
# ones with 16 key / 48 value heads of 128, and the MTP head over the first
# 65536 vocabulary rows (tools/convert_hf.py:225 MTP_DRAFT_VOCAB).
QWEN38 = dict(hidden=5120, n_layer=64, n_heads=24, n_kv_heads=4, head_dim=256, ffn=17408, vocab=248320,
              rms_eps=1e-6, rope_theta=1e7, rot_dim=64, tied=False, hybrid=True,
              layer_types=["linear_attention", "linear_attention", "linear_attention", "full_attention"] * 16,
              lin_nk=16, lin_nv=48, lin_dk=128, lin_dv=128, lin_conv=4, mtp_vocab=65536)


def workload_contexts(n, lo, hi, seed):
    """The benchmark's seeded contexts: n past lengths log-uniform in
    [lo, hi] (configs[2]: 32 chats in [128, 16384], seed 1234)."""
    import math

    import numpy as np
    rng = np.random.default_rng(seed)
    return np.round(np.exp(rng.uniform(math.log(lo), math.log(hi), n))).astype(int)


class Churn:
    """configs[4]'s continuous-batching workload, one pass at a time: `slots`
    chat frames, Poisson(`rate`) arrivals a pass, prompts log-uniform in
    [32, 4096] ids fed as `chunk`-token chunks beside the decode rows (at most
    two chunks a pass, rows <= t_max), chats retiring after U[64, 512]
    generated tokens. Seeded: the same seed gives the same jobs for the same
    sampled ids.

        ch = Churn(vocab, slots=64, chunk=512, t_max=1088, seed=1239)
        jobs = ch.jobs()                # this pass's jobs, in slot order
        done = ch.advance(jobs, ids)    # feed the sampled ids; frames retired
    """

    def __init__(self, vocab, slots, chunk, t_max, seed, rate=2.0, prompt=(32, 4096), stop=(64, 512)):
        import numpy as np
        self.vocab, self.slots, self.chunk, self.t_max = vocab, slots, chunk, t_max
        self.rate, self.prompt, self.stop = rate, prompt, stop
        self.rng = np.random.default_rng(seed)
        self.chats = {}   # frame -> {"prompt", "fed", "gen", "stop", "last"}
        self.stats = {"prefill": 0, "decode": 0, "arrived": 0, "retired": 0, "rows": 0}

    def jobs(self):
        import math
        rng = self.rng
        for _ in range(rng.poisson(self.rate)):
            free = [f for f in range(self.slots) if f not in self.chats]
            if not free:
                break
            lo, hi = self.prompt
            self.chats[free[0]] = {"prompt": int(math.exp(rng.uniform(math.log(lo), math.log(hi)))), "fed": 0,
                                   "gen": 0, "stop": int(rng.integers(self.stop[0], self.stop[1] + 1)), "last": 1}
            self.stats["arrived"] += 1
        jobs, rows, chunks = [], 0, 0
        for f in sorted(self.chats):                  # every decode row
            ch = self.chats[f]
            if ch["fed"] >= ch["prompt"]:
                jobs.append(dict(slot=f, past=ch["fed"], n=1, ids=[ch["last"]], sampled=1))
                rows += 1
        for f in sorted(self.chats):                  # then up to two prompt chunks
            ch = self.chats[f]
            if ch["fed"] < ch["prompt"] and chunks < 2 and rows + self.chunk <= self.t_max:
                n = min(self.chunk, ch["prompt"] - ch["fed"])
                jobs.append(dict(slot=f, past=ch["fed"], n=n,
                                 ids=[(ch["fed"] + i) % self.vocab for i in range(n)],
                                 sampled=1 if ch["fed"] + n == ch["prompt"] else 0))
                rows += n
                chunks += 1
        jobs.sort(key=lambda j: j["slot"])
        return jobs

    def advance(self, jobs, ids):
        """Feeds the pass's sampled ids (one per sampled job, in job order)
        back; returns the frames whose chats retired (the caller releases
        them)."""
        at = 0
        for j in jobs:
            ch = self.chats[j["slot"]]
            self.stats["decode" if ch["fed"] >= ch["prompt"] else "prefill"] += j["n"]
            self.stats["rows"] += j["n"]
            ch["fed"] += j["n"]
            if j["sampled"]:
                ch["last"] = int(ids[at]) % self.vocab
                ch["gen"] += 1
                at += 1
        done = [f for f, ch in self.chats.items() if ch["gen"] >= ch["stop"]]
        for f in done:
            del self.chats[f]
            self.stats["retired"] += 1
        return done
