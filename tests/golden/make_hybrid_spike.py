"""Copies the reference's small Qwen3.5 (hybrid) oracle dump into one fixture.

    python tests/golden/make_hybrid_spike.py /path/to/reference

The arrays are the reference's own data (``oracle/qwen3.8-27b-spike``,
written by its tools/dump_qwen_oracle.py from HF's Qwen3_5 model): one
linear_attention layer's (layer 0) Gated DeltaNet intermediates — the raw
projections, conv in/out, l2-normed q/k, value, gates, the per-token
recurrent states and core output, the gated norm — and one full_attention
layer's (layer 3) q/gate split, q_norm/k_norm, partial-rotary RoPE and
attention output, with the few weights that connect them (conv1d, A_log /
dt_bias, gated_norm, out_proj, q_norm, k_norm, o_proj). They pin
oracle/hybrid.py. Only arrays are read (numpy.load, allow_pickle=False);
nothing of the reference is run. The input projections and the MLP weights
are left out: the fixture starts at the projections' outputs, which keeps it
near 1 MB.
"""
import json
import os
import sys

import numpy as np

NAMES = [
    # layer 0, linear_attention
    "layer00_conv_pre", "layer00_conv_post", "layer00_query_raw", "layer00_key_raw", "layer00_value",
    "layer00_query_l2norm", "layer00_key_l2norm", "layer00_a_raw", "layer00_b_raw", "layer00_A_log",
    "layer00_dt_bias", "layer00_g", "layer00_beta", "layer00_recurrent_core_out_seq",
    "layer00_recurrent_states", "layer00_z_raw", "layer00_gated_norm_out", "layer00_linear_attn_out",
    "weight_layer00_conv1d", "weight_layer00_gated_norm", "weight_layer00_out_proj",
    # layer 3, full_attention
    "layer03_q_proj_raw", "layer03_k_proj_raw", "layer03_v", "layer03_q_norm_out", "layer03_k_norm_out",
    "layer03_q_rope", "layer03_k_rope", "layer03_gate_raw", "layer03_attn_out",
    "weight_layer03_q_norm", "weight_layer03_k_norm", "weight_layer03_o_proj",
]


def main(ref):
    src = os.path.join(ref, "oracle", "qwen3.8-27b-spike")
    arrays = {n: np.load(os.path.join(src, n + ".npy"), allow_pickle=False) for n in NAMES}
    with open(os.path.join(src, "spike_config.json")) as f:
        cfg = json.load(f)
    # tools/dump_qwen_oracle.py builds the model with rms_norm_eps=1e-6
    cfg["rms_norm_eps"] = 1e-6
    arrays["config_json"] = np.frombuffer(json.dumps(cfg, sort_keys=True).encode(), np.uint8)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hybrid_spike.npz")
    np.savez_compressed(out, **arrays)
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
