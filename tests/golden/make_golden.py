"""Writes the whole-forward golden fixtures in tests/golden/ (run once, in the
build container; the committed .npz files are what the tests read).

The fixtures pin the oracle's forward pass independently of the oracle: the
same bf16-rounded weights are loaded into Hugging Face transformers
(Qwen2ForCausalLM / LlamaForCausalLM built from local config objects, f32,
eager attention, no download), and its logits and per-layer residual stream
are stored for a short token sequence.

Cases:
  qwen2_tiny       split-half RoPE, qkv bias, tied embeddings (Config.fromJson shape)
  llama_interleaved interleaved RoPE as VVLI reads GGUF (Config.fromGguf): HF
                   Llama rotates pairs (i, i+hd/2); the q/k rows of every head
                   are permuted so that pair (2i, 2i+1) lands on (i, i+hd/2),
                   which leaves q.k unchanged
  reference_tiny   the reference's own runner-test config (src/llm.zig:1743-1782)
                   with fillDeterministicForTesting f32 weights
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

from vvli_amd import config as C  # noqa: E402
from vvli_amd import runtime as R  # noqa: E402


def blob_to_f32(blob: np.ndarray) -> np.ndarray:
    if blob.dtype == np.uint16:
        return (blob.astype(np.uint32) << 16).view(np.float32)
    return blob.astype(np.float32)


def slices(cfg: C.Config, kind: int) -> dict:
    """Offsets of every tensor (same order as OwnedModel.assignSlices)."""
    ea = 64 // (2 if kind == C.WEIGHT_BF16 else 4)
    h, kv, inter = cfg.hidden_size, cfg.kv_dim(), cfg.intermediate_size
    cur = 0
    out = {}

    def take(name, n):
        nonlocal cur
        cur = (cur + ea - 1) // ea * ea
        out[name] = (cur, n)
        cur += n

    take("embed", cfg.vocab_size * h)
    for l in range(cfg.num_hidden_layers):
        take(f"{l}.input_norm", h)
        take(f"{l}.q", h * h)
        if cfg.qkv_bias:
            take(f"{l}.q_bias", h)
        take(f"{l}.k", kv * h)
        if cfg.qkv_bias:
            take(f"{l}.k_bias", kv)
        take(f"{l}.v", kv * h)
        if cfg.qkv_bias:
            take(f"{l}.v_bias", kv)
        take(f"{l}.o", h * h)
        take(f"{l}.post_norm", h)
        take(f"{l}.gate", inter * h)
        take(f"{l}.up", inter * h)
        take(f"{l}.down", h * inter)
    take("final_norm", h)
    if not cfg.tie_word_embeddings:
        take("lm_head", cfg.vocab_size * h)
    assert cur == cfg.storage_element_count(kind), "layout mismatch with the library"
    return out


def interleave_perm(hd: int) -> np.ndarray:
    """perm[j_hf] = j_ours: HF split-half position of our interleaved index."""
    perm = np.empty(hd, dtype=np.int64)
    for j in range(hd):
        hf = j // 2 if j % 2 == 0 else hd // 2 + (j - 1) // 2
        perm[hf] = j
    return perm


def build_hf(cfg: C.Config, blob: np.ndarray, kind: int, interleaved: bool):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

    common = dict(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                  num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
                  num_key_value_heads=cfg.num_key_value_heads, rms_norm_eps=cfg.rms_norm_eps,
                  max_position_embeddings=cfg.max_position_embeddings,
                  tie_word_embeddings=cfg.tie_word_embeddings,
                  rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta})
    if cfg.architecture == "qwen2":
        hcfg = Qwen2Config(**common)
        model_cls = Qwen2ForCausalLM
    else:
        hcfg = LlamaConfig(attention_bias=cfg.qkv_bias, mlp_bias=False, **common)
        model_cls = LlamaForCausalLM
    hcfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = model_cls(hcfg).float().eval()
    f = blob_to_f32(blob)
    sl = slices(cfg, kind)
    h, kv, hd = cfg.hidden_size, cfg.kv_dim(), cfg.head_dim()

    def t(name, shape):
        off, n = sl[name]
        return torch.from_numpy(f[off:off + n].reshape(shape).copy())

    def rows_perm(w, heads):
        if not interleaved:
            return w
        perm = interleave_perm(hd)
        idx = np.concatenate([hh * hd + perm for hh in range(heads)])
        return w[torch.from_numpy(idx)]

    sd = {"model.embed_tokens.weight": t("embed", (cfg.vocab_size, h)), "model.norm.weight": t("final_norm", (h,))}
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}."
        sd[p + "input_layernorm.weight"] = t(f"{l}.input_norm", (h,))
        sd[p + "post_attention_layernorm.weight"] = t(f"{l}.post_norm", (h,))
        sd[p + "self_attn.q_proj.weight"] = rows_perm(t(f"{l}.q", (h, h)), cfg.num_attention_heads)
        sd[p + "self_attn.k_proj.weight"] = rows_perm(t(f"{l}.k", (kv, h)), cfg.num_key_value_heads)
        sd[p + "self_attn.v_proj.weight"] = t(f"{l}.v", (kv, h))
        sd[p + "self_attn.o_proj.weight"] = t(f"{l}.o", (h, h))
        if cfg.qkv_bias:
            sd[p + "self_attn.q_proj.bias"] = rows_perm(t(f"{l}.q_bias", (h,)), cfg.num_attention_heads)
            sd[p + "self_attn.k_proj.bias"] = rows_perm(t(f"{l}.k_bias", (kv,)), cfg.num_key_value_heads)
            sd[p + "self_attn.v_proj.bias"] = t(f"{l}.v_bias", (kv,))
        sd[p + "mlp.gate_proj.weight"] = t(f"{l}.gate", (cfg.intermediate_size, h))
        sd[p + "mlp.up_proj.weight"] = t(f"{l}.up", (cfg.intermediate_size, h))
        sd[p + "mlp.down_proj.weight"] = t(f"{l}.down", (h, cfg.intermediate_size))
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"] if cfg.tie_word_embeddings else t("lm_head", (cfg.vocab_size, h))
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all(k.endswith("rotary_emb.inv_freq") for k in missing), missing
    return model


def run_hf(model, tokens: np.ndarray, layers: int):
    captured = []
    hooks = [model.model.layers[l].register_forward_hook(
        lambda mod, inp, out: captured.append((out[0] if isinstance(out, tuple) else out).detach().clone()))
        for l in range(layers)]
    with torch.no_grad():
        out = model(torch.from_numpy(tokens.astype(np.int64))[None, :], use_cache=False)
    for hk in hooks:
        hk.remove()
    logits = out.logits[0].float().numpy()
    hidden = torch.stack([c[0] for c in captured], dim=1).float().numpy()  # [T, layers, hidden]
    return logits, hidden


CASES = {
    "qwen2_tiny": dict(
        cfg=C.Config(vocab_size=96, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                     num_key_value_heads=2, max_position_embeddings=64, rope_theta=10_000.0, rms_norm_eps=1e-6,
                     tie_word_embeddings=True, architecture="qwen2", qkv_bias=True, rope_layout=C.ROPE_SPLIT_HALF),
        kind=C.WEIGHT_BF16, how="synth", tokens=12),
    "llama_interleaved": dict(
        cfg=C.Config(vocab_size=80, hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
                     num_key_value_heads=1, max_position_embeddings=64, rope_theta=500_000.0, rms_norm_eps=1e-5,
                     tie_word_embeddings=False, architecture="llama", qkv_bias=False,
                     rope_layout=C.ROPE_INTERLEAVED),
        kind=C.WEIGHT_BF16, how="synth", tokens=12),
    "reference_tiny": dict(cfg=C.tiny_test(), kind=C.WEIGHT_F32, how="det", tokens=8),
}


def main() -> None:
    for name, case in CASES.items():
        cfg, kind = case["cfg"], case["kind"]
        blob = (R.synthetic_blob(cfg, kind, seed=7, stddev=0.15) if case["how"] == "synth"
                else R.deterministic_blob(cfg, kind))
        tokens = np.random.default_rng(11).integers(0, cfg.vocab_size, size=case["tokens"]).astype(np.uint32)
        model = build_hf(cfg, blob, kind, interleaved=cfg.rope_layout == C.ROPE_INTERLEAVED)
        logits, hidden = run_hf(model, tokens, cfg.num_hidden_layers)
        np.savez_compressed(HERE / f"{name}.npz", blob=blob, tokens=tokens, logits=logits, hidden=hidden,
                            weight_kind=np.array(kind))
        print(f"{name}: blob {blob.size} elems, logits {logits.shape}, hidden {hidden.shape}")


if __name__ == "__main__":
    main()
