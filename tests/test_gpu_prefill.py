"""GPU parity of the batched prefill (prefill.hip) with the reference's token
loop (src/generator.zig:243-251), restated by the oracle.

The prefill must leave what the loop leaves: the K/V cache rows of every
prompt position and the logits / argmax of the last prompt token. Bar: K/V
rows and logits within 2e-3 max relative error (max |gpu - ref| / max |ref|),
argmax equal, greedy continuations identical.
"""
import numpy as np
import pytest

from vvli_amd import config as C
from vvli_amd import runtime as R
from vvli_amd._lib import VvliError

pytestmark = pytest.mark.gpu

TOL = 2e-3


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


def cfg_small(**kw) -> C.Config:
    base = dict(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=2, max_position_embeddings=4096, rope_theta=1e6, rms_norm_eps=1e-6,
                tie_word_embeddings=True, architecture="qwen2", qkv_bias=True, rope_layout=C.ROPE_SPLIT_HALF)
    base.update(kw)
    return C.Config(**base)


# name -> (config, blob maker, prompt lengths: one prefill call each, in order)
CASES = {
    # The reference tiny runner config (hd 4 is not a batched shape: token loop).
    "qwen_small": (cfg_small(), "synth", [37]),
    "qwen_small_split": (cfg_small(), "synth", [5, 64, 1, 130]),  # start_pos > 0, ragged tiles
    "llama_small": (cfg_small(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_attention_heads=8,
                              num_key_value_heads=2, qkv_bias=False, tie_word_embeddings=False,
                              architecture="llama", rope_layout=C.ROPE_INTERLEAVED, rope_theta=5e5,
                              rms_norm_eps=1e-5), "synth", [200]),
    "hd128_g7": (cfg_small(vocab_size=640, hidden_size=896, intermediate_size=1024, num_attention_heads=7,
                           num_key_value_heads=1, tie_word_embeddings=False), "synth", [70]),
    # head_dim 128 (32-key tiles) with start_pos > 0: earlier cache rows packed again, ragged last tile.
    "hd128_split": (cfg_small(vocab_size=640, hidden_size=896, intermediate_size=1024, num_attention_heads=7,
                              num_key_value_heads=1, tie_word_embeddings=False), "synth", [45, 3, 97]),
    "qwen05_heads": (cfg_small(vocab_size=2000, hidden_size=896, intermediate_size=4864, num_attention_heads=14,
                               num_key_value_heads=2), "synth", [150]),
    "hd32_g1": (cfg_small(hidden_size=128, num_attention_heads=4, num_key_value_heads=4), "synth", [65]),
    # 1100 rows: ragged GEMM tiles in rows, gate/up columns (2 x 704) and K (704 for down), split K on
    # o_proj / down, 18 row groups of the attention.
    "big_tiles": (cfg_small(hidden_size=512, intermediate_size=704, num_attention_heads=8, num_key_value_heads=2,
                            vocab_size=500), "synth", [1100]),
    # More rows than one chunk (2048): two passes, the second attending to the first's cache rows.
    "two_chunks": (cfg_small(hidden_size=128, intermediate_size=256, num_attention_heads=2, num_key_value_heads=1,
                             vocab_size=300), "synth", [2100]),
}


@pytest.fixture(scope="module")
def built():
    R._lib.lib()
    return True


# Attention-form cases, by the default choice on 256 CUs: 32 kv heads put a
# 600-row prompt on 128-vector blocks with two key groups (160 blocks; the
# 64-vector form would need 320), 64 kv heads a 1100-row prompt on the
# one-group form (576 blocks, more than two rounds).
FORM_CASES = {
    "kv32_two_groups": (cfg_small(vocab_size=500, hidden_size=2048, intermediate_size=512, num_attention_heads=32,
                                  num_key_value_heads=32, qkv_bias=False), "synth", [600]),
    "kv64_one_group": (cfg_small(vocab_size=300, hidden_size=4096, intermediate_size=256, num_attention_heads=64,
                                 num_key_value_heads=64, qkv_bias=False, num_hidden_layers=1), "synth", [1100]),
}


def _check_prefill(name, cfg, parts, oracle_mod, host_threads):
    total = sum(parts)
    max_seq = total + 8
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    toks = np.random.default_rng(11).integers(0, cfg.vocab_size, size=total).astype(np.uint32)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_prefill_path("batched")
        start = 0
        for n in parts:
            logits, am = gpu.prefill(toks[start:start + n], start)
            logits = logits.copy()
            for i in range(start, start + n):
                ref = orc.forward_token(int(toks[i]), i)
            e = rel_err(logits, ref)
            assert e <= TOL, f"{name} prefill [{start}, {start + n}): logits rel err {e:.3e}"
            assert am == oracle_mod.argmax(ref)
            start += n
        for layer in range(cfg.num_hidden_layers):
            for pos in sorted({0, 1, total // 3, total // 2, total - 2, total - 1}):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"{name} kv layer {layer} pos {pos}"
        # The next token step continues from the prefilled state.
        nxt = int(toks[0])
        e = rel_err(gpu.forward_token(nxt, total), orc.forward_token(nxt, total))
        assert e <= TOL, f"{name} step after prefill: {e:.3e}"


@pytest.mark.parametrize("form", [0, 1, 2])
@pytest.mark.parametrize("name", ["qwen_small_split", "llama_small", "hd128_split", "hd32_g1"])
def test_attention_forms_match_token_loop(name, form, built, oracle_mod, host_threads):
    """Every launch form of the prefill attention (blocks of 128 query
    vectors with one or two key groups, blocks of 64 with two), forced through
    the test hook, against the token loop: ragged tiles, start_pos > 0,
    head_dim 32 / 64 / 128, groups 1 / 2 / 4 / 7."""
    cfg, how, parts = CASES[name]
    lib = R._lib.lib()
    print(f"case={name} parts={parts} attention form {form}", flush=True)
    R._lib.check(lib.vvli_gpu_test_set_prefill_attention_form(form))
    try:
        _check_prefill(name, cfg, parts, oracle_mod, host_threads)
    finally:
        R._lib.check(lib.vvli_gpu_test_set_prefill_attention_form(-1))


@pytest.mark.parametrize("name", list(FORM_CASES))
def test_attention_default_forms_match_token_loop(name, built, oracle_mod, host_threads):
    cfg, how, parts = FORM_CASES[name]
    print(f"case={name} parts={parts}", flush=True)
    _check_prefill(name, cfg, parts, oracle_mod, host_threads)


@pytest.mark.parametrize("name", list(CASES))
def test_batched_prefill_matches_token_loop(name, built, oracle_mod, host_threads):
    cfg, how, parts = CASES[name]
    total = sum(parts)
    max_seq = total + 8
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    toks = np.random.default_rng(11).integers(0, cfg.vocab_size, size=total).astype(np.uint32)
    print(f"case={name} parts={parts}", flush=True)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_prefill_path("batched")
        start = 0
        for n in parts:
            logits, am = gpu.prefill(toks[start:start + n], start)
            logits = logits.copy()
            for i in range(start, start + n):
                ref = orc.forward_token(int(toks[i]), i)
            e = rel_err(logits, ref)
            assert e <= TOL, f"{name} prefill [{start}, {start + n}): logits rel err {e:.3e}"
            assert am == oracle_mod.argmax(ref)
            start += n
        for layer in range(cfg.num_hidden_layers):
            for pos in sorted({0, 1, total // 3, total // 2, total - 2, total - 1}):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"{name} kv layer {layer} pos {pos}"
        # The next token step continues from the prefilled state.
        nxt = int(toks[0])
        e = rel_err(gpu.forward_token(nxt, total), orc.forward_token(nxt, total))
        assert e <= TOL, f"{name} step after prefill: {e:.3e}"


@pytest.mark.parametrize("path", ["graph", "persistent"])
@pytest.mark.parametrize("name", ["qwen_small", "llama_small", "hd128_g7"])
def test_generate_with_batched_prefill(name, path, built, oracle_mod, host_threads):
    cfg, how, parts = CASES[name]
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02)
    n_prompt, n_new = 48, 40
    prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, size=n_prompt).astype(np.uint32)
    orc = oracle_mod.OracleRunner(cfg, blob, 128, threads=host_threads)
    ref, _ = orc.generate_greedy(prompt, n_new)
    print(f"case={name} path={path}", flush=True)
    with R.Runner(cfg, blob, 128) as gpu:
        gpu.set_decode_path(path)
        got, stats = gpu.generate_greedy_measured(prompt, n_new, batched_prefill=True)
        assert stats.prompt_tokens == n_prompt and stats.generated_tokens == n_new
        np.testing.assert_array_equal(got, ref)
        gpu.kv_clear()
        eos = int(ref[n_new // 2])
        first = int(np.argmax(ref == eos))
        got2, _ = gpu.generate_greedy_measured(prompt, n_new, eos_token_id=eos, batched_prefill=True)
        np.testing.assert_array_equal(got2, ref[: first + 1])


def test_prefill_paths_and_errors(built):
    lib = R._lib.lib()
    assert lib.vvli_gpu_test_set_prefill_attention_form(3) == 1
    assert lib.vvli_gpu_test_set_prefill_attention_form(-2) == 1
    tiny = C.tiny_test()  # head_dim 4: the token loop serves it
    with R.Runner(tiny, R.deterministic_blob(tiny, C.WEIGHT_BF16), 16) as gpu:
        with pytest.raises(VvliError):
            gpu.set_prefill_path("batched")
        gpu.set_prefill_path("auto")
        gpu.prefill([1, 2, 3])
    cfg = cfg_small()
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0)
    with R.Runner(cfg, blob, 32) as gpu:
        gpu.set_prefill_path("batched")
        with pytest.raises(VvliError) as e:
            gpu.prefill(np.arange(20), 20)  # 20 + 20 > max_seq_len 32
        assert e.value.name == "ContextFull"
        with pytest.raises(VvliError) as e:
            gpu.prefill([cfg.vocab_size])
        assert e.value.name == "InvalidToken"
        with pytest.raises(VvliError) as e:
            gpu.prefill([])
        assert e.value.name == "EmptyPrompt"
        # Batched and token-loop prefill agree with each other too.
        toks = np.random.default_rng(1).integers(0, cfg.vocab_size, size=30)
        lb, ab = gpu.prefill(toks)
        lb = lb.copy()
        gpu.kv_clear()
        gpu.set_prefill_path("loop")
        ll, al = gpu.prefill(toks)
        assert ab == al and rel_err(lb, ll) <= TOL
