"""Copies the reference's own weight-free golden vectors into tests/golden/.

    python tests/golden/make_golden.py /path/to/reference

These are data files the reference's tests hold (HF intermediates dumped by
its tools/dump_*_oracle.py and read by web/dev/verify.js): a block's q/k
projections before RoPE and the split-half RoPE of them computed in f64, plus
the Qwen spike's cos/sin table. They pin the oracle's RoPE table and rotation
(oracle/ccoracle.c orc_rope_table / orc_rope) without any weights. Block 0's
residual-stream dumps (the embedding rows, both norms' outputs, the attention
and MLP sublayers' outputs, the residual between them and the block's output)
pin the block's composition (oracle/model.py compose_block) the same way.
Only arrays are copied (numpy.load with allow_pickle=False); nothing is run.
"""
import json
import os
import sys

import numpy as np

FILES = {
    # reference path (under oracle/) -> fixture name
    "smollm2/block00_q.npy": "smollm2_q.npy",
    "smollm2/block00_q_rope.npy": "smollm2_q_rope.npy",
    "smollm2/block00_k.npy": "smollm2_k.npy",
    "smollm2/block00_k_rope.npy": "smollm2_k_rope.npy",
    "llama-3.1-8b-instruct/block00_q.npy": "llama31_q.npy",
    "llama-3.1-8b-instruct/block00_q_rope.npy": "llama31_q_rope.npy",
    "llama-3.1-8b-instruct/block00_k.npy": "llama31_k.npy",
    "llama-3.1-8b-instruct/block00_k_rope.npy": "llama31_k_rope.npy",
    "qwen3.8-27b-spike/rope_cos.npy": "qwen_spike_rope_cos.npy",
    # block 0's residual stream (HF, f32): embeddings -> ln1 -> attention ->
    # +residual -> ln2 -> MLP -> +residual
    **{f"{src}/{a}.npy": f"{dst}_{b}.npy"
       for src, dst in (("smollm2", "smollm2"), ("llama-3.1-8b-instruct", "llama31"))
       for a, b in (("embeddings", "embeddings"), ("block00_ln1", "ln1"), ("block00_attn_out", "attn_out"),
                    ("block00_after_attn_resid", "after_attn_resid"), ("block00_ln2", "ln2"),
                    ("block00_mlp_out", "mlp_out"), ("block_00_out", "block_out"))},
    "qwen3.8-27b-spike/rope_sin.npy": "qwen_spike_rope_sin.npy",
}

# The RoPE settings each fixture was produced with: SmolLM2's config
# (web/model/kernels.js:23-37 DIMS: theta 1e5, head_dim 64), Llama 3.1's
# published config (theta 5e5, "llama3" scaling factor 8, low 1, high 4,
# original 8192; tools/dump_llama_oracle.py:41-51 reads it from HF), and the
# Qwen spike's spike_config.json (theta 1e7, head_dim 64, rot 16).
PARAMS = {
    "smollm2": {"theta": 100000.0, "head_dim": 64, "n_heads": 9, "n_kv_heads": 3, "rot": 64, "rms_eps": 1e-5},
    "llama31": {"theta": 500000.0, "head_dim": 128, "n_heads": 32, "n_kv_heads": 8, "rot": 128, "rms_eps": 1e-5,
                "scaling": {"factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                            "original_max_position_embeddings": 8192}},
    "qwen_spike": {"theta": 10000000.0, "head_dim": 64, "rot": 16},
}


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    here = os.path.dirname(os.path.abspath(__file__))
    for src, dst in FILES.items():
        a = np.load(os.path.join(ref, "oracle", src), allow_pickle=False)
        np.save(os.path.join(here, dst), a, allow_pickle=False)
    with open(os.path.join(here, "rope_params.json"), "w") as f:
        json.dump(PARAMS, f, indent=2)
    print(f"wrote {len(FILES)} fixtures to {here}")


if __name__ == "__main__":
    main()
