"""Writes tests/golden/olmoe_tiny.npz: a mixture-of-experts golden fixture
(run once, in the build container; the committed .npz is what tests read).

The reference has no MoE forward pass, so the MoE step follows HF
transformers' OLMoE. This script builds a tiny OlmoeForCausalLM from a local
config object (no download), sets every parameter from a seeded generator and
rounds it to bf16, runs the token sequence through it in f32 with eager
attention, and stores the weights (bf16 bits, HF names), the tokens, the
logits of every position, the residual stream after every layer but the last,
and the experts the router picks at every (position, layer).

Weights: linear and embedding N(0, 0.05); router N(0, 0.5) so the routing
probabilities are well separated; RMSNorm weights 1 + N(0, 0.1) so the norm
weights are exercised.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
import transformers

HERE = Path(__file__).resolve().parent

CONFIG = dict(vocab_size=96, hidden_size=64, intermediate_size=32, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=2, max_position_embeddings=64, rms_norm_eps=1e-5, num_experts=8,
              num_experts_per_tok=2, tie_word_embeddings=False, norm_topk_prob=False, rope_theta=10000.0,
              eos_token_id=1, pad_token_id=0, bos_token_id=0)
TOKENS = [3, 17, 42, 5, 88, 17, 60, 9]


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    cfg = transformers.OlmoeConfig(**CONFIG)
    cfg._attn_implementation = "eager"
    model = transformers.OlmoeForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(1234)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                v = 1.0 + 0.1 * torch.randn(p.shape, generator=g)
            elif name.endswith("mlp.gate.weight"):
                v = 0.5 * torch.randn(p.shape, generator=g)
            else:
                v = 0.05 * torch.randn(p.shape, generator=g)
            p.copy_(v.to(torch.bfloat16).float())
    ids = torch.tensor([TOKENS], dtype=torch.long)
    picks = []
    hooks = [layer.mlp.gate.register_forward_hook(lambda mod, inp, out: picks.append(out[2].clone()))
             for layer in model.model.layers]
    with torch.no_grad():
        out = model(ids, output_hidden_states=True)
    for h in hooks:
        h.remove()
    L = cfg.num_hidden_layers
    experts = torch.stack(picks, dim=1).numpy().astype(np.uint32)  # [pos, layer, k] (router order)
    hidden = torch.stack(out.hidden_states[1:L], dim=2)[0].numpy().astype(np.float32)  # [pos, L-1, H]
    arrays = {f"w/{k}": bf16_bits(v) for k, v in model.state_dict().items()}
    arrays.update(
        tokens=np.array(TOKENS, dtype=np.uint32),
        logits=out.logits[0].numpy().astype(np.float32),
        hidden=hidden,
        experts=experts,
        config=np.frombuffer(json.dumps(CONFIG).encode(), dtype=np.uint8),
    )
    np.savez_compressed(HERE / "olmoe_tiny.npz", **arrays)
    print("wrote", HERE / "olmoe_tiny.npz", {k: v.shape for k, v in arrays.items() if not k.startswith("w/")})


if __name__ == "__main__":
    main()
