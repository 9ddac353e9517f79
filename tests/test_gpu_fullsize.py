"""Full-size parity: the benchmark workloads' real shapes (Qwen2.5-0.5B,
Llama-3.2-1B, Qwen2.5-7B, OLMoE-1B-7B) with seeded synthetic bf16 weights,
against the oracle on the same blob.

Bar: the residual stream after every layer and the logits
within 2e-3 max relative error for the first positions, and the greedy tokens
identical. Sequence lengths are cut to what the CPU oracle finishes in
seconds; the GPU runs the same code paths the benchmark runs (persistent
decode step, batched prefill)."""
import os

import numpy as np
import pytest

from vvli_amd import config as C
from vvli_amd import gguf_write
from vvli_amd import loaders as L
from vvli_amd import runtime as R

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

TOL = 2e-3


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


def bf16_bits(a: np.ndarray) -> np.ndarray:
    b = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


# name -> (config, prompt tokens, greedy tokens, positions checked layer by layer)
DENSE = {
    "qwen2.5-0.5b": (C.qwen25_05b(), 32, 64, 3),
    "llama-3.2-1b": (C.llama32_1b(), 32, 64, 3),
    "qwen2.5-7b": (C.qwen25_7b(), 16, 32, 2),
}


@pytest.mark.parametrize("name", list(DENSE))
def test_dense_full_size(name, oracle_mod, host_threads):
    cfg, n_prompt, n_new, n_check = DENSE[name]
    max_seq = 512
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02, threads=host_threads)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    print(f"case={name} layer parity", flush=True)
    with R.Runner(cfg, blob, max_seq) as gpu:
        for pos in range(n_check):
            ref_logits, ref_hidden = orc.forward_token(int(prompt[pos]), pos, want_hidden=True)
            logits, hidden = gpu.forward_token_debug(int(prompt[pos]), pos)
            worst = max(rel_err(hidden[l], ref_hidden[l]) for l in range(cfg.num_hidden_layers))
            assert worst <= TOL, f"{name} pos {pos}: hidden rel err {worst:.3e}"
            assert rel_err(logits, ref_logits) <= TOL, f"{name} pos {pos}: logits"
        orc.kv_clear()
        gpu.kv_clear()
        ref, _ = orc.generate_greedy(prompt, n_new)
        print(f"case={name} greedy {n_prompt}+{n_new}", flush=True)
        got, _ = gpu.generate_greedy_measured(prompt, n_new, batched_prefill=True)
        np.testing.assert_array_equal(got, ref)


def test_olmoe_full_size(oracle_mod, host_threads):
    cfg = C.olmoe_1b_7b()
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02, threads=host_threads)
    lay = oracle_mod.moe_layout(cfg, C.WEIGHT_BF16)
    rng = np.random.default_rng(100)
    n = cfg.num_experts * cfg.hidden_size
    for L in lay["layers"]:  # router logits ~ N(0, 1) on unit-RMS input
        blob[L["router"]:L["router"] + n] = bf16_bits(rng.normal(0, 1 / np.sqrt(cfg.hidden_size), n))
    # The MoE workload: 64 prompt tokens, 64 decoded.
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, 64).astype(np.uint32)
    orc = oracle_mod.OracleMoeRunner(cfg, blob, 160, threads=host_threads)
    print("case=olmoe-1b-7b", flush=True)
    with R.MoeRunner(cfg, blob, 160) as gpu:
        for pos in range(2):
            ref_logits, ref_hidden, _ = orc.forward_token(int(prompt[pos]), pos, want_hidden=True)
            logits, hidden = gpu.forward_token_debug(int(prompt[pos]), pos)
            worst = max(rel_err(hidden[l], ref_hidden[l]) for l in range(cfg.num_hidden_layers))
            assert worst <= TOL, f"pos {pos}: hidden rel err {worst:.3e}"
            assert rel_err(logits, ref_logits) <= TOL
        gpu.kv_clear()
        orc2 = oracle_mod.OracleMoeRunner(cfg, blob, 160, threads=host_threads)
        ref = orc2.generate_greedy(prompt, 64)
        got, _ = gpu.generate_greedy_measured(prompt, 64)
        np.testing.assert_array_equal(got, ref)


def test_llama1b_workload_as_benched(oracle_mod, host_threads, tmp_path):
    """The headline decode workload exactly as bench.py times it: Llama-3.2-1B
    shape (16 layers), seeded N(0, 0.02) bf16 weights written as a GGUF file
    and loaded through the device GGUF loader, the llama3-scaled RoPE table,
    a 512-token batched prefill, then 128 greedy tokens from one persistent
    decode launch at ctx 4096 (generator.zig's loop: src/generator.zig:221-293).

    Bar: the 128 tokens identical to the oracle's (its prompt runs token by
    token, as the reference does), and the residual stream after every layer
    and the logits within 2e-3 at positions 512, 575 and 639 (each step
    recomputed on both sides over the KV cache the generation left)."""
    cfg = C.llama32_1b()
    ctx, n_prompt, n_new = 4096, 512, 128
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02, threads=host_threads)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
    table = R.llama3_inv_freq(cfg.head_dim(), cfg.rope_theta)
    path = os.path.join(tmp_path, "llama-3.2-1b.gguf")
    gguf_write.write_dense_gguf(path, cfg, blob)
    print("case=llama-3.2-1b workload: GGUF -> device loader, 512 + 128, ctx 4096", flush=True)
    gcfg, gpu = L.device_load_gguf(path, ctx)
    os.remove(path)
    with gpu:
        assert gcfg.num_hidden_layers == 16 and gcfg.rope_layout == C.ROPE_INTERLEAVED
        gpu.set_decode_path("persistent")
        gpu.set_rope_table(table)
        got, stats = gpu.generate_greedy_measured(prompt, n_new, batched_prefill=True)
        assert stats.generated_tokens == n_new
        orc = oracle_mod.OracleRunner(cfg, blob, ctx, threads=host_threads)
        orc.set_rope_table(table)
        print("case=llama-3.2-1b workload: oracle 512 + 128", flush=True)
        ref, _ = orc.generate_greedy(prompt, n_new)
        np.testing.assert_array_equal(got, ref)
        for pos in (512, 575, 639):  # token fed at pos: the (pos - 512)-th generated one
            tok = int(ref[pos - n_prompt])
            ref_logits, ref_hidden = orc.forward_token(tok, pos, want_hidden=True)
            logits, hidden = gpu.forward_token_debug(tok, pos)
            worst = max(rel_err(hidden[l], ref_hidden[l]) for l in range(cfg.num_hidden_layers))
            assert worst <= TOL, f"pos {pos}: hidden rel err {worst:.3e}"
            assert rel_err(logits, ref_logits) <= TOL, f"pos {pos}: logits"


def test_qwen7b_long_context_full_size(oracle_mod, host_threads):
    """The Qwen2.5-7B workload's decode at its real length: a 4096-token
    batched prefill at ctx 8192 (two 2048-row chunks) on the GPU; the
    oracle's prompt pass over the first 128 tokens (their K/V rows at the
    32-key tile edges compared in every layer); then the oracle continues
    from the GPU's cache (all 4096 rows of every layer copied in) through
    eight persistent decode steps at positions 4096-4103: every layer's
    residual, the logits, the argmax and
    the new K/V rows against the oracle. At these positions each kv head has
    43 attention splits (spread merge, matrix-core tiles), and the down phase
    stages the 18944-wide SwiGLU vector. The full prompt pass is out of the
    oracle's reach (about 60 TFLOP on the host), hence the copied cache."""
    cfg = C.qwen25_7b()
    ctx, n_prompt, n_head, n_steps = 8192, 4096, 128, 8
    L_, kv = cfg.num_hidden_layers, cfg.kv_dim()
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02, threads=host_threads)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
    orc = oracle_mod.OracleRunner(cfg, blob, ctx, threads=host_threads)
    print("case=qwen2.5-7b long context: 4096-token prefill", flush=True)
    with R.Runner(cfg, blob, ctx) as gpu:
        gpu.set_prefill_path("batched")
        gpu.set_decode_path("persistent")
        _, am = gpu.prefill(prompt, 0)
        print(f"case=qwen2.5-7b long context: oracle prompt pass over {n_head} tokens", flush=True)
        orc.prefill(prompt[:n_head], 0)
        for layer in range(L_):
            for pos in (0, 31, 32, 63, 64, 95, 96, n_head - 1):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"kv layer {layer} pos {pos}"
        print("case=qwen2.5-7b long context: cache copied to the oracle", flush=True)
        k = np.empty((n_prompt, kv), np.float32)
        v = np.empty((n_prompt, kv), np.float32)
        for layer in range(L_):
            for pos in range(n_prompt):
                k[pos], v[pos] = gpu.kv_read(layer, pos)
            orc.kv_write(layer, 0, k, v)
        tok = int(am)
        for step in range(n_steps):
            pos = n_prompt + step
            print(f"case=qwen2.5-7b long context: step at pos {pos}", flush=True)
            ref_logits, ref_hidden = orc.forward_token(tok, pos, want_hidden=True)
            logits, hidden = gpu.forward_token_debug(tok, pos)
            worst = max(rel_err(hidden[l], ref_hidden[l]) for l in range(L_))
            assert worst <= TOL, f"pos {pos}: hidden rel err {worst:.3e}"
            assert rel_err(logits, ref_logits) <= TOL, f"pos {pos}: logits"
            assert R.argmax(logits) == oracle_mod.argmax(ref_logits), f"pos {pos}: argmax"
            for layer in (0, L_ // 2, L_ - 1):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"new kv row layer {layer} pos {pos}"
            tok = oracle_mod.argmax(ref_logits)
