"""Parity of the shipped decode path at the lengths it is timed at.

The persistent step (the default decode path) is checked layer by layer --
the residual stream after every layer, written by its down-projection phases
(vvli_gpu_forward_token_debug on the persistent path) -- against the oracle
(the CPU restatement of src/llm.zig:732-766 and computeAttentionInto,
:1302-1335), after a batched prefill of the prompt, at the attention
geometries of the two long-context workloads:

* Llama-3.2-1B heads (hidden 2048, 32 q / 8 kv heads, head_dim 64,
  interleaved RoPE): 512-token prompt, then 128 decode steps at ctx 4096, so
  positions 512..639 merge 9 and 10 attention splits of 64 positions; with the
  reference RoPE and with the llama3-scaled table.
* Qwen2.5-7B heads (hidden 3584, 28 q / 4 kv heads, head_dim 128, group 7,
  qkv bias, untied): 4096-token prompt, then 256 decode steps at ctx 8192, so
  every step merges 43..46 splits of 96 positions (each split merging at most
  21 of its head's 896 outputs; at 46 splits one merges none).
* The spread merge at head_dim 64 beyond 16 splits: Llama-3.2-1B heads at
  positions 2016-2055 (32 splits, each merging 8 of its kv head's 256
  outputs, then 17 splits of 128 positions) with the llama3 table, and
  Qwen2.5-0.5B heads (14 q / 2 kv, group 7) at positions 4064-4095 (64
  splits, each merging 7 of its kv head's 448 outputs).

Two layers, and a reduced intermediate size and vocabulary, keep the oracle's
CPU time to seconds; the attention shapes, the split counts and the KV lengths
are the workloads' own. Bar: per-layer residuals and logits within 2e-3 max
relative error, the same argmax every step (the oracle's argmax is fed back as
the next token), KV rows within 2e-3.
"""
import numpy as np
import pytest

from vvli_amd import config as C
from vvli_amd import runtime as R

pytestmark = pytest.mark.gpu

TOL = 2e-3


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


def cfg_llama1b_heads() -> C.Config:
    return C.Config(vocab_size=2048, hidden_size=2048, intermediate_size=1024, num_hidden_layers=2,
                    num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072, rope_theta=5e5,
                    rms_norm_eps=1e-5, tie_word_embeddings=True, architecture="llama", qkv_bias=False,
                    rope_layout=C.ROPE_INTERLEAVED)


def cfg_qwen7b_heads() -> C.Config:
    return C.Config(vocab_size=512, hidden_size=3584, intermediate_size=512, num_hidden_layers=2,
                    num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=32768, rope_theta=1e6,
                    rms_norm_eps=1e-6, tie_word_embeddings=False, architecture="qwen2", qkv_bias=True,
                    rope_layout=C.ROPE_SPLIT_HALF)


def splits_at(pos: int, max_seq: int, kv_heads: int, head_dim: int, blocks: int = 256) -> int:
    """Attention splits the persistent step merges at `pos` (its split rule:
    at most min(64, ceil(max_seq / 64), blocks / kv_heads) splits of at least
    64 positions, a whole number of K/V tiles each -- 64 rows at head_dim <= 64,
    32 at 128; blocks: one per CU, 256 on an MI355X)."""
    nsplit = max(1, min(64, (max_seq + 63) // 64, blocks // kv_heads))
    tile = 64 if head_dim <= 64 else 32
    t = pos + 1
    chunk = max(64, -(-t // nsplit))
    chunk = -(-chunk // tile) * tile
    return -(-t // chunk)


def cfg_qwen05b_heads() -> C.Config:
    return C.Config(vocab_size=512, hidden_size=896, intermediate_size=512, num_hidden_layers=2,
                    num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=32768, rope_theta=1e6,
                    rms_norm_eps=1e-6, tie_word_embeddings=True, architecture="qwen2", qkv_bias=True,
                    rope_layout=C.ROPE_SPLIT_HALF)


CASES = {
    # name: (config maker, ctx, prompt, decode steps, llama3 table)
    "llama1b_heads_512p128": (cfg_llama1b_heads, 4096, 512, 128, False),
    "llama1b_heads_512p128_llama3rope": (cfg_llama1b_heads, 4096, 512, 128, True),
    "qwen7b_heads_4096p256": (cfg_qwen7b_heads, 8192, 4096, 256, False),
    # Llama-3.2-1B heads past position 1024: 32 splits of 64 positions up to
    # position 2047, then 17 of 128 -- the spread merge at head_dim 64.
    "llama1b_heads_2016p40": (cfg_llama1b_heads, 4096, 2016, 40, True),
    # Qwen2.5-0.5B heads (14 q / 2 kv, head_dim 64, group 7): 64 splits at
    # positions 4032-4095, the most the step uses.
    "qwen05b_heads_4064p32": (cfg_qwen05b_heads, 8192, 4064, 32, False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_persistent_decode_long_context(name, oracle_mod, host_threads):
    make, ctx, n_prompt, steps, llama3 = CASES[name]
    cfg = make()
    L = cfg.num_hidden_layers
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab_size, size=n_prompt).astype(np.uint32)
    want_splits = sorted({splits_at(p, ctx, cfg.num_key_value_heads, cfg.head_dim())
                          for p in range(n_prompt, n_prompt + steps)})
    print(f"case={name} prompt={n_prompt} steps={steps} ctx={ctx} splits={want_splits}", flush=True)
    orc = oracle_mod.OracleRunner(cfg, blob, ctx, threads=host_threads)
    with R.Runner(cfg, blob, ctx) as gpu:
        gpu.set_decode_path("persistent")
        gpu.set_prefill_path("batched")
        if llama3:
            table = R.llama3_inv_freq(cfg.head_dim(), cfg.rope_theta)
            gpu.set_rope_table(table)
            orc.set_rope_table(table)
        ref = orc.prefill(prompt)
        got, am = gpu.prefill(prompt)
        e = rel_err(got, ref)
        assert e <= TOL, f"{name} prefill last logits rel err {e:.3e}"
        assert am == oracle_mod.argmax(ref), f"{name} prefill argmax"
        tok = oracle_mod.argmax(ref)
        worst = 0.0
        for s in range(steps):
            pos = n_prompt + s
            ref, ref_hidden = orc.forward_token(tok, pos, want_hidden=True)
            got, hidden = gpu.forward_token_debug(tok, pos)
            for layer in range(L):
                e = rel_err(hidden[layer], ref_hidden[layer])
                worst = max(worst, e)
                assert e <= TOL, f"{name} pos {pos} layer {layer}: hidden rel err {e:.3e}"
            e = rel_err(got, ref)
            worst = max(worst, e)
            assert e <= TOL, f"{name} pos {pos}: logits rel err {e:.3e}"
            nxt = oracle_mod.argmax(ref)
            assert R.argmax(got) == nxt, f"{name} pos {pos}: argmax"
            tok = nxt
        last = n_prompt + steps - 1
        for layer in range(L):
            for pos in (0, n_prompt // 2, n_prompt - 1, n_prompt, last):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"{name} kv layer {layer} pos {pos}"
        print(f"case={name} worst rel err {worst:.2e}", flush=True)
