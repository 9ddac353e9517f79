"""Writes tests/golden/llama3_rope.npz: Llama-3 RoPE frequency tables computed
by Hugging Face transformers' _compute_llama3_parameters (a third-party
implementation of the published closed form; the reference has no RoPE
scaling) for the rope_scaling blocks of Llama-3.2 and Llama-3.1. Run once in
the build container; the tests read the committed file."""
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

CASES = {
    # name: (head_dim, theta, factor, low_freq_factor, high_freq_factor, original_max_pos)
    "llama32": (64, 500000.0, 32.0, 1.0, 4.0, 8192),
    "llama31": (128, 500000.0, 8.0, 1.0, 4.0, 8192),
}


def main() -> None:
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import _compute_llama3_parameters

    out = {}
    for name, (hd, theta, factor, lo, hi, orig) in CASES.items():
        cfg = LlamaConfig(hidden_size=hd * 4, num_attention_heads=4, head_dim=hd,
                          rope_parameters={"rope_type": "llama3", "rope_theta": theta, "factor": factor,
                                           "low_freq_factor": lo, "high_freq_factor": hi,
                                           "original_max_position_embeddings": orig})
        inv, _ = _compute_llama3_parameters(cfg, "cpu")
        out[name] = inv.numpy().astype(np.float32)
        out[name + "_params"] = np.array([hd, theta, factor, lo, hi, orig], dtype=np.float64)
        print(name, out[name][:3], out[name][-3:])
    np.savez_compressed(HERE / "llama3_rope.npz", **out)


if __name__ == "__main__":
    main()
