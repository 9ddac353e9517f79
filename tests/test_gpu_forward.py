"""GPU parity of the token step against the oracle (CPU restatement of the
reference forward pass, oracle/vvli_oracle.c), through the C ABI.

Bar: per-layer residual stream and logits within 2e-3 max relative error
(max |gpu - ref| / max |ref|, f32 accumulation on both sides), K/V cache rows
within the same bound, greedy token sequences identical.
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


# name -> (config, weight kind, blob maker, positions to step through)
CASES = {
    # The reference's own tiny runner test (src/llm.zig:1743-1782), f32 and bf16 blobs.
    "tiny_f32": (C.tiny_test(), C.WEIGHT_F32, "det", 8),
    "tiny_bf16": (C.tiny_test(), C.WEIGHT_BF16, "det", 8),
    # Qwen2-style: split-half RoPE, qkv bias, tied, hd 64, GQA group 2.
    "qwen_small": (cfg_small(), C.WEIGHT_BF16, "synth", 70),
    # Llama-from-GGUF style: interleaved RoPE, no bias, untied, GQA group 4.
    "llama_small": (cfg_small(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_attention_heads=8,
                              num_key_value_heads=2, qkv_bias=False, tie_word_embeddings=False,
                              architecture="llama", rope_layout=C.ROPE_INTERLEAVED, rope_theta=5e5,
                              rms_norm_eps=1e-5), C.WEIGHT_BF16, "synth", 40),
    # hd 128, group 7 (the Qwen2.5-7B head shape).
    "hd128_g7": (cfg_small(vocab_size=640, hidden_size=896, intermediate_size=1024, num_attention_heads=7,
                           num_key_value_heads=1, tie_word_embeddings=False), C.WEIGHT_BF16, "synth", 40),
    # Qwen2.5-0.5B head shape: hidden 896, 14/2 heads, K = 896 and 4864.
    "qwen05_heads": (cfg_small(vocab_size=2000, hidden_size=896, intermediate_size=4864, num_attention_heads=14,
                               num_key_value_heads=2), C.WEIGHT_BF16, "synth", 24),
    # f32 weights through the f32 kernel variants.
    "qwen_small_f32": (cfg_small(), C.WEIGHT_F32, "synth", 20),
    # head_dim 96 (between the 64 and 128 kernels: the head-dim-128 persistent
    # kernel with its columns d >= 96 masked), GQA group 4, interleaved RoPE.
    "hd96_g4": (cfg_small(vocab_size=700, hidden_size=768, intermediate_size=1024, num_attention_heads=8,
                          num_key_value_heads=2, qkv_bias=False, architecture="llama",
                          rope_layout=C.ROPE_INTERLEAVED), C.WEIGHT_BF16, "synth", 40),
}


def make_blob(cfg, kind, how):
    if how == "det":
        return R.deterministic_blob(cfg, kind)
    return R.synthetic_blob(cfg, kind, seed=0, stddev=0.02)


@pytest.fixture(scope="module")
def built():
    R._lib.lib()
    return True


STEP_CASES = [(n, "graph") for n in CASES] + [(n, "persistent") for n in CASES if CASES[n][1] == C.WEIGHT_BF16]


@pytest.mark.parametrize("name,path", STEP_CASES)
def test_token_steps_match_oracle(name, path, built, oracle_mod, host_threads):
    """Per-layer residuals and logits of every step, on the per-kernel step
    ('graph': the kernels launched eagerly) and on the persistent step (its
    down-projection phases write the residual rows)."""
    cfg, kind, how, steps = CASES[name]
    max_seq = min(cfg.max_position_embeddings, 128)
    blob = make_blob(cfg, kind, how)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    rng = np.random.default_rng(1)
    toks = rng.integers(0, cfg.vocab_size, size=steps)
    print(f"case={name} path={path} steps={steps}", flush=True)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_decode_path(path)
        for pos, tok in enumerate(toks):
            ref_logits, ref_hidden = orc.forward_token(int(tok), pos, want_hidden=True)
            logits, hidden = gpu.forward_token_debug(int(tok), pos)
            for layer in range(cfg.num_hidden_layers):
                e = rel_err(hidden[layer], ref_hidden[layer])
                assert e <= TOL, f"{name} pos {pos} layer {layer}: hidden rel err {e:.3e}"
            e = rel_err(logits, ref_logits)
            assert e <= TOL, f"{name} pos {pos}: logits rel err {e:.3e}"
        for layer in range(cfg.num_hidden_layers):
            for pos in (0, steps // 2, steps - 1):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"{name} kv layer {layer} pos {pos}"


@pytest.mark.parametrize("name", ["tiny_f32", "qwen_small", "llama_small"])
def test_graph_step_equals_debug_step(name, built):
    """The graph-replayed per-kernel step (forward_token on the 'graph' path)
    gives the same logits and argmax as the eagerly launched one
    (forward_token_debug): same kernels, same order."""
    cfg, kind, how, steps = CASES[name]
    blob = make_blob(cfg, kind, how)
    max_seq = min(cfg.max_position_embeddings, 64)
    toks = np.random.default_rng(2).integers(0, cfg.vocab_size, size=min(steps, 12))
    with R.Runner(cfg, blob, max_seq) as a, R.Runner(cfg, blob, max_seq) as b:
        a.set_decode_path("graph")
        b.set_decode_path("graph")  # forward_token_debug then launches the same kernels eagerly
        for pos, tok in enumerate(toks):
            la = a.forward_token(int(tok), pos).copy()
            am = a.last_argmax
            lb, _ = b.forward_token_debug(int(tok), pos)
            np.testing.assert_array_equal(la, lb)
            assert am == R.argmax(la)


BF16_CASES = ["tiny_bf16", "qwen_small", "llama_small", "hd128_g7", "qwen05_heads", "hd96_g4"]


@pytest.mark.parametrize("name", BF16_CASES)
def test_persistent_steps_match_oracle(name, built, oracle_mod, host_threads):
    """The one-launch persistent step (forward_token on the 'persistent'
    path): logits, argmax and K/V rows against the oracle, token by token."""
    cfg, kind, how, steps = CASES[name]
    # llama_small (head_dim 64), hd128_g7 (head_dim 128, the matrix-core
    # tile) and hd96_g4 (the same tile with masked columns): 2 splits of 64
    # positions (every split merges a slice of the outputs) up to 5 (the
    # appending split merges the others).
    steps = {"llama_small": 300, "hd128_g7": 300, "hd96_g4": 300}.get(name, steps)
    max_seq = min(cfg.max_position_embeddings, 512)
    blob = make_blob(cfg, kind, how)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    toks = np.random.default_rng(1).integers(0, cfg.vocab_size, size=steps)
    print(f"case={name} steps={steps} persistent", flush=True)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_decode_path("persistent")
        for pos, tok in enumerate(toks):
            ref = orc.forward_token(int(tok), pos)
            got = gpu.forward_token(int(tok), pos)
            e = rel_err(got, ref)
            assert e <= TOL, f"{name} pos {pos}: logits rel err {e:.3e}"
            assert gpu.last_argmax == oracle_mod.argmax(ref), f"{name} pos {pos}: argmax"
        for layer in range(cfg.num_hidden_layers):
            for pos in (0, steps - 1):
                gk, gv = gpu.kv_read(layer, pos)
                rk, rv = orc.kv_read(layer, pos)
                assert rel_err(gk, rk) <= TOL and rel_err(gv, rv) <= TOL, f"{name} kv layer {layer} pos {pos}"


@pytest.mark.parametrize("path", ["graph", "persistent"])
@pytest.mark.parametrize("name", ["qwen_small", "llama_small"])
def test_forward_token_return_forms_match_oracle(name, path, built, oracle_mod, host_threads):
    """The three ways a per-token caller reads a step: logits copied into its
    buffer, the borrowed view of the library's pinned logits (the reference's
    slice return, src/llm.zig:729), and the argmax only -- interleaved over
    consecutive positions, each against the oracle. The view keeps its
    address, is read-only, and holds the latest call's logits."""
    cfg, kind, how, _ = CASES[name]
    blob = make_blob(cfg, kind, how)
    orc = oracle_mod.OracleRunner(cfg, blob, 128, threads=host_threads)
    toks = np.random.default_rng(3).integers(0, cfg.vocab_size, size=30)
    print(f"case={name} path={path} return forms", flush=True)
    addr = None
    with R.Runner(cfg, blob, 128) as gpu:
        gpu.set_decode_path(path)
        for pos, tok in enumerate(toks):
            ref = orc.forward_token(int(tok), pos)
            form = pos % 3
            if form == 0:
                got = gpu.forward_token(int(tok), pos)
                assert rel_err(got, ref) <= TOL, f"{name} pos {pos}: logits"
                am = gpu.last_argmax
            elif form == 1:
                view = gpu.forward_token_view(int(tok), pos)
                assert not view.flags.writeable and view.size == cfg.vocab_size
                a = view.__array_interface__["data"][0]
                assert addr is None or a == addr, "the view moved"
                addr = a
                assert rel_err(view, ref) <= TOL, f"{name} pos {pos}: view logits"
                am = gpu.last_argmax
                assert am == R.argmax(view)
            else:
                am = gpu.forward_token_argmax(int(tok), pos)
            assert am == oracle_mod.argmax(ref), f"{name} pos {pos} form {form}: argmax"


@pytest.mark.parametrize("path", ["graph", "persistent"])
def test_forward_token_up_to_the_last_position(path, built, oracle_mod, host_threads):
    """Single steps at every position up to max_seq_len - 1 (the step at the
    last position also marks the cache full), then ContextFull
    (src/llm.zig:706-707) at max_seq_len; the argmax-only form at the last
    position."""
    cfg, kind, how, _ = CASES["qwen_small"]
    max_seq = 48
    blob = make_blob(cfg, kind, how)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    toks = np.random.default_rng(8).integers(0, cfg.vocab_size, size=max_seq)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_decode_path(path)
        for pos in range(max_seq - 1):
            ref = orc.forward_token(int(toks[pos]), pos)
            got = gpu.forward_token(int(toks[pos]), pos)
            assert rel_err(got, ref) <= TOL and gpu.last_argmax == oracle_mod.argmax(ref), f"pos {pos}"
        ref = orc.forward_token(int(toks[-1]), max_seq - 1)
        assert gpu.forward_token_argmax(int(toks[-1]), max_seq - 1) == oracle_mod.argmax(ref)
        with pytest.raises(VvliError) as e:
            gpu.forward_token(int(toks[0]), max_seq)
        assert e.value.rc == 4


@pytest.mark.parametrize("path", ["graph", "persistent"])
@pytest.mark.parametrize("name", ["tiny_bf16", "qwen_small", "llama_small", "hd128_g7"])
def test_greedy_generation_matches_oracle(name, path, built, oracle_mod, host_threads):
    cfg, kind, how, _ = CASES[name]
    blob = make_blob(cfg, kind, how)
    max_seq = min(cfg.max_position_embeddings, 96)
    n_prompt = min(8, max_seq // 2)
    n_new = max_seq - n_prompt
    prompt = np.random.default_rng(3).integers(0, cfg.vocab_size, size=n_prompt).astype(np.uint32)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    ref, _ = orc.generate_greedy(prompt, n_new)
    print(f"case={name} path={path}", flush=True)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_decode_path(path)
        got, stats = gpu.generate_greedy_measured(prompt, n_new)
        assert stats.generated_tokens == n_new and stats.prompt_tokens == n_prompt
        np.testing.assert_array_equal(got, ref)
        # Same run with EOS = a token that appears mid-sequence stops right after it.
        gpu.kv_clear()
        eos = int(ref[n_new // 2])
        first = int(np.argmax(ref == eos))
        got2, stats2 = gpu.generate_greedy_measured(prompt, n_new, eos_token_id=eos)
        np.testing.assert_array_equal(got2, ref[: first + 1])


def test_forward_embedding_matches_oracle(built, oracle_mod):
    cfg, kind, how, _ = CASES["qwen_small"]
    blob = make_blob(cfg, kind, how)
    orc = oracle_mod.OracleRunner(cfg, blob, 16, threads=2)
    emb = np.full(cfg.hidden_size, 0.01, dtype=np.float32)  # src/llm.zig:1777-1778
    with R.Runner(cfg, blob, 16) as gpu:
        gpu.forward_token(3, 0)
        orc.forward_token(3, 0)
        got = gpu.forward_embedding(emb, 1).copy()
        ref = orc.forward_embedding(emb, 1)
        assert rel_err(got, ref) <= TOL
        assert np.isfinite(got).all()


def test_runner_errors(built):
    cfg = C.tiny_test()
    blob = R.deterministic_blob(cfg, C.WEIGHT_F32)
    with R.Runner(cfg, blob, 8) as gpu:
        with pytest.raises(VvliError) as e:
            gpu.forward_token(cfg.vocab_size, 0)  # src/llm.zig:704
        assert e.value.name == "InvalidToken"
        with pytest.raises(VvliError) as e:
            gpu.forward_token(1, 8)  # src/llm.zig:705
        assert e.value.name == "ContextFull"
        with pytest.raises(VvliError) as e:
            gpu.generate_greedy_measured(np.zeros(0, dtype=np.uint32), 4)  # src/generator.zig:230
        assert e.value.name == "EmptyPrompt"
        with pytest.raises(VvliError) as e:
            gpu.generate_greedy_measured(np.zeros(4, dtype=np.uint32), 8)  # 4 + 8 > 8 positions
        assert e.value.name == "ContextFull"
        # The runner still works after the errors.
        assert np.isfinite(gpu.forward_token(3, 0)).all()


@pytest.mark.parametrize("path", ["graph", "persistent"])
def test_llama3_rope_table_matches_oracle(path, built, oracle_mod, host_threads):
    """A Llama-3 scaled RoPE table (vvli_host_llama3_inv_freq, pinned against
    Hugging Face in the CPU tests) set on both sides: token steps agree."""
    cfg, kind, how, _ = CASES["llama_small"]
    blob = make_blob(cfg, kind, how)
    table = R.llama3_inv_freq(cfg.head_dim(), cfg.rope_theta, factor=32.0, low_freq_factor=1.0,
                              high_freq_factor=4.0, original_max_pos=64)  # a short original context: every band used
    orc = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
    orc.set_rope_table(table)
    toks = np.random.default_rng(5).integers(0, cfg.vocab_size, size=24)
    print(f"llama3 rope path={path}", flush=True)
    with R.Runner(cfg, blob, 64) as gpu:
        gpu.set_decode_path(path)
        gpu.set_rope_table(table)
        for pos, tok in enumerate(toks):
            ref = orc.forward_token(int(tok), pos)
            got = gpu.forward_token(int(tok), pos)
            e = rel_err(got, ref)
            assert e <= TOL, f"pos {pos}: logits rel err {e:.3e}"
        # Clearing the table restores the reference formula.
        gpu.set_rope_table(None)
        gpu.kv_clear()
        for pos, tok in enumerate(toks[:8]):
            plain = gpu.forward_token(int(tok), pos).copy()
        orc2 = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
        for pos, tok in enumerate(toks[:8]):
            ref_plain = orc2.forward_token(int(tok), pos)
        assert rel_err(plain, ref_plain) <= TOL


def test_persistent_error_flag_is_reported(built, oracle_mod, host_threads):
    """The persistent step's failure path, forced from the host
    (vvli_gpu_test_inject_step_error): a launch that starts with its error
    flag raised leaves before any phase and the waiting call returns
    VVLI_HIP_ERROR; the runner works afterwards. In the sampled generation
    loop, which checks the flag only at its end, a flag raised in a middle
    launch is still reported (later launches must not clear it)."""
    cfg, kind, how, _ = CASES["qwen_small"]
    blob = make_blob(cfg, kind, how)
    lib = R._lib.lib()
    toks = [5, 77, 300, 12]
    orc = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
    orc_ref1 = None
    print("inject: forward_token", flush=True)
    with R.Runner(cfg, blob, 64) as gpu:
        gpu.set_decode_path("persistent")
        gpu.forward_token(toks[0], 0)
        R._lib.check(lib.vvli_gpu_test_inject_step_error(gpu._h, 1))
        with pytest.raises(VvliError) as e:
            gpu.forward_token(toks[1], 1)
        assert e.value.rc == 8 and "injected" in str(e.value)
        # The flag was read and cleared: the step runs again and the runner continues.
        for pos in range(len(toks)):
            ref = orc.forward_token(toks[pos], pos)
            if pos == 1:
                orc_ref1 = ref.copy()
            if pos == 0:
                continue
            got = gpu.forward_token(toks[pos], pos)
            assert rel_err(got, ref) <= TOL and gpu.last_argmax == oracle_mod.argmax(ref)
        # The same on the argmax-only and view calls (no logits copy).
        for call in (gpu.forward_token_argmax, gpu.forward_token_view):
            R._lib.check(lib.vvli_gpu_test_inject_step_error(gpu._h, 1))
            with pytest.raises(VvliError) as e:
                call(toks[1], 1)
            assert e.value.rc == 8 and "injected" in str(e.value)
            out = call(toks[1], 1)
            am = out if isinstance(out, int) else gpu.last_argmax
            assert am == oracle_mod.argmax(orc_ref1)
    print("inject: sampled generation, third per-token launch", flush=True)
    prompt = np.array(toks, dtype=np.uint32)
    opts = R.Sampling(temperature=0.8, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, seed=7)
    with R.Runner(cfg, blob, 64) as gpu:
        gpu.set_decode_path("persistent")
        R._lib.check(lib.vvli_gpu_test_inject_step_error(gpu._h, 3))
        with pytest.raises(VvliError) as e:
            gpu.generate(prompt, 8, opts, batched_prefill=True)
        assert e.value.rc == 8
        gpu.kv_clear()
        got, _ = gpu.generate(prompt, 8, opts, batched_prefill=True)
    ref_orc = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
    want = ref_orc.generate_sampled(prompt, 8, opts)
    np.testing.assert_array_equal(got, want)
    print("inject: greedy generation, decode launch", flush=True)
    with R.Runner(cfg, blob, 64) as gpu:
        gpu.set_decode_path("persistent")
        R._lib.check(lib.vvli_gpu_test_inject_step_error(gpu._h, 2))  # 1: the prompt launch, 2: decode
        with pytest.raises(VvliError) as e:
            gpu.generate_greedy_measured(prompt, 8)
        assert e.value.rc == 8
