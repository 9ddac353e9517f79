"""Pins the oracle (oracle/vvli_oracle.c, the CPU restatement of the
reference forward pass) before the GPU parity tests rely on it.

Each check is something the oracle's own formula cannot satisfy by
construction: the reference's inline-test known answers, f64 brute force,
closed forms and special cases, and whole-forward golden fixtures computed by
an independent implementation (HF transformers, tests/golden/make_golden.py).
"""
import math
from pathlib import Path

import numpy as np
import pytest

from vvli_amd import config as C
from vvli_amd import runtime as R

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------------------
# Reference known answers (the reference's own inline tests)
# ---------------------------------------------------------------------------
def test_rope_known_answer(oracle_mod):
    # src/llm.zig:1703-1716: pos 1, theta 1e4, head_dim 4, input [1,2,3,4].
    v = np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float32)
    split = oracle_mod.rope(v, 1, 4, 1, 10_000.0, C.ROPE_SPLIT_HALF)
    inter = oracle_mod.rope(v, 1, 4, 1, 10_000.0, C.ROPE_INTERLEAVED)
    c, s = math.cos(1.0), math.sin(1.0)
    assert abs(split[0] - (1 * c - 3 * s)) <= 1e-6
    assert abs(split[2] - (1 * s + 3 * c)) <= 1e-6
    assert abs(inter[0] - (1 * c - 2 * s)) <= 1e-6
    assert abs(inter[1] - (1 * s + 2 * c)) <= 1e-6


def test_rmsnorm_known_answer(oracle_mod):
    # src/tensor.zig:866-878: [3, 4], w = 1, eps = 0 -> [0.84852815, 1.1313708].
    out = oracle_mod.rmsnorm(np.array([3.0, 4.0], np.float32), np.array([1.0, 1.0], np.float32), 0.0)
    assert abs(out[0] - 0.84852815) <= 1e-6 and abs(out[1] - 1.1313708) <= 1e-6


def test_matmul_known_answer(oracle_mod):
    # src/tensor.zig:793-812: [[1,2,3],[4,5,6]] . [[7,8],[9,10],[11,12]] = [58,64,139,154].
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    rows = [oracle_mod.linear(np.ascontiguousarray(b.T), a[m]) for m in range(2)]
    assert np.array_equal(np.concatenate(rows), np.array([58, 64, 139, 154], np.float32))


def test_softmax_known_answers(oracle_mod):
    # src/tensor.zig:848-864: a row sums to 1; a uniform row gives 1/3.
    assert abs(oracle_mod.softmax(np.array([1, 2, 3], np.float32)).sum() - 1.0) <= 1e-6
    assert np.allclose(oracle_mod.softmax(np.array([1, 1, 1], np.float32)), 1 / 3, atol=1e-6)


def test_bf16_round_trip(oracle_mod):
    # src/llm.zig:1690-1701 within 0.01, plus exact RNE bit patterns.
    for v in (1.0, -2.5, 0.25, 8.0):
        assert abs(oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(v)) - v) <= 0.01
    assert oracle_mod.f32_to_bf16(1.0) == 0x3F80
    # 1 + 2^-8 is a tie between 0x3F80 and 0x3F81: RNE keeps the even 0x3F80.
    assert oracle_mod.f32_to_bf16(1.0 + 2**-8) == 0x3F80
    # 1 + 3*2^-8 ties between 0x3F81 and 0x3F82: RNE goes to the even 0x3F82.
    assert oracle_mod.f32_to_bf16(1.0 + 3 * 2**-8) == 0x3F82
    assert oracle_mod.f32_to_bf16(1.0 + 2**-8 + 2**-16) == 0x3F81


def test_greedy_with_repeat_penalty(oracle_mod):
    # src/generator.zig:491-499: logits [10, 9.8, 1], counts [1,0,0], penalty 2 -> token 1.
    lib = oracle_mod.lib()
    logits = np.array([10.0, 9.8, 1.0], np.float32)
    counts = np.array([1, 0, 0], np.uint16)
    tok = lib.orc_greedy_with_penalties(oracle_mod._p(logits), oracle_mod._p(counts), 3, 2.0)
    assert tok == 1
    assert lib.orc_greedy_with_penalties(oracle_mod._p(logits), oracle_mod._p(counts), 3, 1.0) == 0


def test_throughput_math():
    # src/generator.zig:470-480: 4 tokens in 2 s -> 2 tok/s.
    st = R.Stats(3, 4, 10**9, 2 * 10**9, 3 * 10**9)
    assert st.decode_tokens_per_second() == 2.0


# ---------------------------------------------------------------------------
# Shape contract (src/llm.zig:1579-1741)
# ---------------------------------------------------------------------------
QWEN_JSON = """{"model_type": "qwen2", "vocab_size": 151936, "hidden_size": 896, "intermediate_size": 4864,
 "num_hidden_layers": 24, "num_attention_heads": 14, "num_key_value_heads": 2, "max_position_embeddings": 32768,
 "rope_theta": 1000000.0, "rms_norm_eps": 1e-6, "tie_word_embeddings": true, "eos_token_id": 151645,
 "pad_token_id": 151654}"""


def test_qwen_config_counts(oracle_mod):
    cfg = C.Config.from_json(QWEN_JSON)
    assert (cfg.head_dim(), cfg.kv_dim(), cfg.kv_group_size()) == (64, 128, 7)
    assert cfg.parameter_count() > 494_005_120
    assert cfg.parameter_count() == oracle_mod.parameter_count(cfg) == 494_032_768
    assert cfg.storage_element_count(C.WEIGHT_BF16) >= cfg.parameter_count()
    assert cfg.storage_element_count(C.WEIGHT_BF16) * 2 < cfg.storage_element_count(C.WEIGHT_F32) * 4
    assert cfg.qkv_bias and cfg.rope_layout == C.ROPE_SPLIT_HALF


def test_llama_and_mistral_configs():
    llama = C.Config.from_json("""{"model_type": "llama", "vocab_size": 128256, "hidden_size": 2048,
        "intermediate_size": 8192, "num_hidden_layers": 16, "num_attention_heads": 32, "num_key_value_heads": 8,
        "max_position_embeddings": 131072, "rope_theta": 500000.0, "rms_norm_eps": 1e-5,
        "tie_word_embeddings": true, "attention_bias": false, "eos_token_id": 128009, "pad_token_id": 128004}""")
    assert llama.architecture == "llama" and llama.num_experts == 0 and llama.head_dim() == 64
    mistral = C.Config.from_json("""{"model_type": "mistral", "vocab_size": 32000, "hidden_size": 4096,
        "intermediate_size": 14336, "num_hidden_layers": 32, "num_attention_heads": 32, "num_key_value_heads": 8,
        "max_position_embeddings": 32768, "rope_theta": 10000.0, "rms_norm_eps": 1e-5,
        "tie_word_embeddings": false, "eos_token_id": 2, "pad_token_id": 2}""")
    assert mistral.rope_layout == C.ROPE_SPLIT_HALF and not mistral.qkv_bias


def test_olmoe_rejected_by_dense_runner():
    # src/llm.zig:1660-1688: parses as MoE; OwnedModel.init -> UnsupportedModelArchitecture.
    cfg = C.Config.from_json("""{"model_type": "olmoe", "vocab_size": 50304, "hidden_size": 2048,
        "intermediate_size": 1024, "num_hidden_layers": 16, "num_attention_heads": 16, "num_key_value_heads": 16,
        "num_experts": 64, "num_experts_per_tok": 8, "max_position_embeddings": 4096, "rope_theta": 10000.0,
        "rms_norm_eps": 1e-5, "tie_word_embeddings": false, "attention_bias": false, "eos_token_id": 50279,
        "pad_token_id": 1}""")
    assert cfg.num_experts == 64 and cfg.qk_norm
    blob = np.zeros(16, np.uint16)
    with pytest.raises(R._lib.VvliError) as e:
        R.Runner(cfg, blob, 16)  # rejected before any device work
    assert e.value.name == "UnsupportedModelArchitecture"


def test_config_errors():
    with pytest.raises(R._lib.VvliError) as e:
        C.Config.from_json('{"model_type": "qwen2", "vocab_size": 10}')
    assert e.value.name == "MissingJsonField"
    with pytest.raises(R._lib.VvliError) as e:
        C.Config.from_json('{"model_type": "gpt2"}')
    assert e.value.name == "UnsupportedModelArchitecture"
    bad = C.tiny_test()
    bad.num_key_value_heads = 3  # heads % kv_heads != 0
    with pytest.raises(R._lib.VvliError) as e:
        bad.validate()
    assert e.value.name == "InvalidConfig"


@pytest.mark.parametrize("kind", [C.WEIGHT_F32, C.WEIGHT_BF16])
def test_blob_layout_alignment_and_agreement(oracle_mod, kind):
    # src/llm.zig:1718-1741 and assignSlices: every slice on a 64-byte boundary,
    # library and oracle agree on every offset, norms land where the layout says.
    rng = np.random.default_rng(5)
    ea = 32 if kind == C.WEIGHT_BF16 else 16
    for _ in range(20):
        heads = int(rng.choice([1, 2, 4, 8]))
        kvh = int(rng.choice([h for h in (1, 2, 4, 8) if heads % h == 0]))
        hd = int(rng.choice([2, 4, 6, 8]))
        cfg = C.Config(vocab_size=int(rng.integers(3, 70)), hidden_size=heads * hd,
                       intermediate_size=int(rng.integers(1, 50)), num_hidden_layers=int(rng.integers(1, 4)),
                       num_attention_heads=heads, num_key_value_heads=kvh, max_position_embeddings=8,
                       rope_theta=1e4, rms_norm_eps=1e-6, tie_word_embeddings=bool(rng.integers(0, 2)),
                       qkv_bias=bool(rng.integers(0, 2)))
        lay = oracle_mod.layout(cfg, kind)
        assert lay["total"] == cfg.storage_element_count(kind)
        assert lay["total"] * (2 if kind else 4) >= cfg.parameter_count() * (2 if kind else 4)
        offs = [lay["embed"], lay["final_norm"]] + [v for L in lay["layers"] for v in L.values() if v is not None]
        assert all(o % ea == 0 for o in offs)
        if kind == C.WEIGHT_BF16:
            blob = R.synthetic_blob(cfg, kind, seed=1)
            norm_offs = [lay["final_norm"]] + [o for L in lay["layers"] for o in (L["input_norm"], L["post_norm"])]
            for o in norm_offs:
                assert np.all(blob[o:o + cfg.hidden_size] == 0x3F80)  # RMSNorm weights = 1.0


def test_fill_deterministic_matches(oracle_mod):
    cfg = C.tiny_test()
    for kind in (C.WEIGHT_F32, C.WEIGHT_BF16):
        a = R.deterministic_blob(cfg, kind)
        b = oracle_mod.fill_deterministic(a.size, kind)
        assert np.array_equal(a, b)
        i = np.arange(a.size)
        expect = ((i % 251) - 125).astype(np.float32) * np.float32(0.001)
        got = (a.astype(np.uint32) << 16).view(np.float32) if kind else a
        assert np.allclose(got, expect, atol=0.001 * 2**-7 * 130)


# ---------------------------------------------------------------------------
# Closed forms / f64 brute force
# ---------------------------------------------------------------------------
def bf16_bits(x: np.ndarray) -> np.ndarray:
    b = x.astype(np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("lanes", [1, 4, 8, 16])
@pytest.mark.parametrize("kind", ["f32", "bf16"])
def test_linear_matches_f64(oracle_mod, lanes, kind):
    rng = np.random.default_rng(lanes)
    for rows, cols in [(7, 5), (33, 64), (16, 1000), (3, 4099)]:
        w32 = rng.normal(0, 0.05, size=(rows, cols)).astype(np.float32)
        x = rng.normal(0, 1, size=cols).astype(np.float32)
        bias = rng.normal(0, 0.1, size=rows).astype(np.float32)
        if kind == "bf16":
            w = bf16_bits(w32)
            wf = (w.astype(np.uint32) << 16).view(np.float32)
            b = bf16_bits(bias)
            bf = (b.astype(np.uint32) << 16).view(np.float32)
        else:
            w, wf, b, bf = w32, w32, bias, bias
        got = oracle_mod.linear(w, x, b, lanes=lanes)
        ref = wf.astype(np.float64) @ x.astype(np.float64) + bf.astype(np.float64)
        scale = np.abs(wf).astype(np.float64) @ np.abs(x).astype(np.float64) + 1
        assert np.all(np.abs(got - ref) <= 4e-7 * math.sqrt(cols) * scale), (rows, cols)
        # A transposed or row-shifted weight would not pass.
        assert not np.allclose(got, np.roll(ref, 1), atol=1e-3)


def test_rope_matches_f64_closed_form(oracle_mod):
    rng = np.random.default_rng(2)
    for layout in (C.ROPE_INTERLEAVED, C.ROPE_SPLIT_HALF):
        for hd, pos, theta in [(8, 0, 1e4), (64, 37, 1e6), (128, 4000, 5e5), (6, 5, 1e4)]:
            heads = 3
            v = rng.normal(size=heads * hd).astype(np.float32)
            got = oracle_mod.rope(v, heads, hd, pos, theta, layout)
            ref = v.astype(np.float64).copy()
            for h in range(heads):
                base = h * hd
                for i in range(hd // 2):
                    a, b = (base + 2 * i, base + 2 * i + 1) if layout == C.ROPE_INTERLEAVED else (base + i, base + i + hd // 2)
                    inv = 1.0 / float(np.float32(theta) ** np.float32(np.float32(2 * i) / np.float32(hd)))
                    ang = float(np.float32(np.float32(pos) * np.float32(inv)))
                    x0, x1 = float(v[a]), float(v[b])
                    ref[a] = x0 * math.cos(ang) - x1 * math.sin(ang)
                    ref[b] = x0 * math.sin(ang) + x1 * math.cos(ang)
            assert np.max(np.abs(got - ref)) <= 1e-5 * (1 + np.max(np.abs(ref))), (layout, hd, pos)


def test_attention_matches_f64(oracle_mod):
    rng = np.random.default_rng(3)
    for heads, kvh, hd, pos in [(4, 2, 8, 0), (4, 2, 8, 9), (7, 1, 16, 30), (8, 8, 4, 3)]:
        kvw = kvh * hd
        q = rng.normal(size=heads * hd).astype(np.float32)
        keys = rng.normal(size=(pos + 1, kvw)).astype(np.float32)
        vals = rng.normal(size=(pos + 1, kvw)).astype(np.float32)
        got = oracle_mod.attention(q, keys, vals, heads, kvh, hd, pos)
        ref = np.zeros(heads * hd)
        g = heads // kvh
        for h in range(heads):
            kh = h // g
            s = keys[:, kh * hd:(kh + 1) * hd].astype(np.float64) @ q[h * hd:(h + 1) * hd].astype(np.float64)
            s /= math.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            ref[h * hd:(h + 1) * hd] = p @ vals[:, kh * hd:(kh + 1) * hd].astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-5, (heads, kvh, hd, pos)


def test_rmsnorm_silu_add_closed_forms(oracle_mod):
    rng = np.random.default_rng(4)
    x = rng.normal(size=1000).astype(np.float32)
    w = rng.normal(size=1000).astype(np.float32)
    got = oracle_mod.rmsnorm(x, w, 1e-5)
    ref = x.astype(np.float64) * w / math.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    assert np.max(np.abs(got - ref)) <= 1e-5
    g = rng.normal(size=257).astype(np.float32) * 5
    u = rng.normal(size=257).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.max(np.abs(oracle_mod.silu_mul(g, u) - ref)) <= 1e-5


def test_argmax_special_cases(oracle_mod):
    # First index of the strict maximum (src/llm.zig:778-789).
    assert oracle_mod.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle_mod.argmax(np.array([-0.0, 0.0, -1.0], np.float32)) == 0
    assert oracle_mod.argmax(np.array([1.0, np.nan, 2.0], np.float32)) == 2
    assert oracle_mod.argmax(np.array([np.nan, 5.0, 7.0], np.float32)) == 0
    assert oracle_mod.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


# ---------------------------------------------------------------------------
# Whole forward against independent golden fixtures
# ---------------------------------------------------------------------------
def golden_cfg(name):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.CASES[name]["cfg"]


@pytest.mark.parametrize("name", ["qwen2_tiny", "llama_interleaved", "reference_tiny"])
def test_oracle_forward_matches_golden(oracle_mod, name):
    data = np.load(GOLDEN / f"{name}.npz")
    cfg = golden_cfg(name)
    blob, tokens = data["blob"], data["tokens"]
    orc = oracle_mod.OracleRunner(cfg, blob, cfg.max_position_embeddings, threads=2)
    for pos, tok in enumerate(tokens):
        logits, hidden = orc.forward_token(int(tok), pos, want_hidden=True)
        ref_l, ref_h = data["logits"][pos], data["hidden"][pos]
        scale = np.max(np.abs(ref_l))
        assert np.max(np.abs(logits - ref_l)) <= 2e-5 * scale + 1e-6, f"{name} pos {pos} logits"
        for layer in range(cfg.num_hidden_layers):
            hs = np.max(np.abs(ref_h[layer]))
            assert np.max(np.abs(hidden[layer] - ref_h[layer])) <= 2e-5 * hs + 1e-6, f"{name} pos {pos} layer {layer}"


def test_golden_detects_wrong_rope_layout(oracle_mod):
    """A planted mistake in the oracle's input (the other RoPE layout) must
    fail the same comparison, or the fixture would pin nothing about RoPE."""
    data = np.load(GOLDEN / "llama_interleaved.npz")
    cfg = golden_cfg("llama_interleaved")
    cfg.rope_layout = C.ROPE_SPLIT_HALF
    orc = oracle_mod.OracleRunner(cfg, data["blob"], cfg.max_position_embeddings, threads=2)
    errs = []
    for pos, tok in enumerate(data["tokens"]):
        logits = orc.forward_token(int(tok), pos)
        errs.append(np.max(np.abs(logits - data["logits"][pos])) / np.max(np.abs(data["logits"][pos])))
    assert max(errs) > 1e-3


def test_reference_tiny_runner_test(oracle_mod):
    # src/llm.zig:1743-1782: logits finite, argmax in range; forwardEmbedding too.
    cfg = C.tiny_test()
    blob = R.deterministic_blob(cfg, C.WEIGHT_F32)
    orc = oracle_mod.OracleRunner(cfg, blob, 8, threads=2)
    logits = orc.forward_token(3, 0)
    assert logits.size == cfg.vocab_size and np.isfinite(logits).all()
    assert oracle_mod.argmax(logits) < cfg.vocab_size
    emb = orc.forward_embedding(np.full(16, 0.01, np.float32), 1)
    assert np.isfinite(emb).all()
    with pytest.raises(oracle_mod.OracleError):
        orc.forward_token(cfg.vocab_size, 0)  # InvalidToken
    with pytest.raises(oracle_mod.OracleError):
        orc.forward_token(1, 8)  # ContextFull


def test_generator_loop_replays_forward_steps(oracle_mod):
    """orc_generate_greedy equals a manual forward/argmax replay (the loop of
    generateGreedy, src/generator.zig:142-175) including forwarding the last token."""
    data = np.load(GOLDEN / "qwen2_tiny.npz")
    cfg = golden_cfg("qwen2_tiny")
    a = oracle_mod.OracleRunner(cfg, data["blob"], 40, threads=2)
    toks, st = a.generate_greedy(data["tokens"][:5], 20)
    b = oracle_mod.OracleRunner(cfg, data["blob"], 40, threads=2)
    for pos, t in enumerate(data["tokens"][:5]):
        logits = b.forward_token(int(t), pos)
    manual = []
    pos = 5
    for _ in range(20):
        nxt = oracle_mod.argmax(logits)
        manual.append(nxt)
        logits = b.forward_token(nxt, pos)
        pos += 1
    assert list(toks) == manual
    assert st.generated_tokens == 20 and st.prompt_tokens == 5
    # EOS stops right after the first occurrence.
    eos = manual[7]
    c = oracle_mod.OracleRunner(cfg, data["blob"], 40, threads=2)
    toks2, _ = c.generate_greedy(data["tokens"][:5], 20, eos=eos)
    assert list(toks2) == manual[: manual.index(eos) + 1]


@pytest.mark.parametrize("case", ["tiny_f32", "qwen_bf16", "llama_bf16_untied"])
def test_prefill_pass_equals_token_loop(oracle_mod, case):
    """orc_prefill (the prompt loop with its loops interchanged, used for the
    long-prompt GPU cases) leaves bit-identical KV rows and last logits to one
    orc_forward_token per token, over two calls (start_pos > 0) that cross
    token blocks and thread boundaries unevenly."""
    if case == "tiny_f32":
        import dataclasses

        cfg, kind = dataclasses.replace(C.tiny_test(), max_position_embeddings=64), C.WEIGHT_F32
        blob = R.deterministic_blob(cfg, kind)
    else:
        kw = dict(vocab_size=300, hidden_size=128, intermediate_size=192, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128, rope_theta=1e6,
                  rms_norm_eps=1e-6, tie_word_embeddings=True, architecture="qwen2", qkv_bias=True,
                  rope_layout=C.ROPE_SPLIT_HALF)
        if case == "llama_bf16_untied":
            kw.update(qkv_bias=False, tie_word_embeddings=False, architecture="llama",
                      rope_layout=C.ROPE_INTERLEAVED, rms_norm_eps=1e-5, num_attention_heads=8)
        cfg, kind = C.Config(**kw), C.WEIGHT_BF16
        blob = R.synthetic_blob(cfg, kind, seed=5)
    toks = np.random.default_rng(9).integers(0, cfg.vocab_size, size=53)
    n1 = 37
    loop = oracle_mod.OracleRunner(cfg, blob, 64, threads=3)
    for pos, t in enumerate(toks):
        want = loop.forward_token(int(t), pos)
        if pos == n1 - 1:
            want_mid = want
    batch = oracle_mod.OracleRunner(cfg, blob, 64, threads=5)
    got_mid = batch.prefill(toks[:n1], 0)
    got = batch.prefill(toks[n1:], n1)
    assert np.array_equal(got_mid.view(np.uint32), want_mid.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for layer in range(cfg.num_hidden_layers):
        for pos in range(len(toks)):
            a, b = batch.kv_read(layer, pos), loop.kv_read(layer, pos)
            assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)), (layer, pos)
            assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32)), (layer, pos)
    # The next token step continues from the same state.
    nxt = oracle_mod.argmax(want)
    assert np.array_equal(batch.forward_token(nxt, len(toks)).view(np.uint32),
                          loop.forward_token(nxt, len(toks)).view(np.uint32))


def test_kv_write_continues_like_the_computed_cache(oracle_mod):
    """orc_kv_write (the setter the full-size long-context GPU test uses to
    continue from the GPU's cache): a runner whose cache rows are copied from
    another's continues with bit-identical logits and rows; a wrong row
    changes the next step; out-of-range rows are rejected."""
    kw = dict(vocab_size=300, hidden_size=128, intermediate_size=192, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=2, max_position_embeddings=64, rope_theta=1e6, rms_norm_eps=1e-6,
              tie_word_embeddings=True, architecture="qwen2", qkv_bias=True, rope_layout=C.ROPE_SPLIT_HALF)
    cfg = C.Config(**kw)
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=3)
    toks = np.random.default_rng(4).integers(0, cfg.vocab_size, size=12)
    a = oracle_mod.OracleRunner(cfg, blob, 32, threads=2)
    for pos, t in enumerate(toks[:10]):
        a.forward_token(int(t), pos)
    b = oracle_mod.OracleRunner(cfg, blob, 32, threads=2)
    for layer in range(cfg.num_hidden_layers):
        rows = [a.kv_read(layer, pos) for pos in range(10)]
        b.kv_write(layer, 0, np.stack([r[0] for r in rows]), np.stack([r[1] for r in rows]))
    want = a.forward_token(int(toks[10]), 10)
    got = b.forward_token(int(toks[10]), 10)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for layer in range(cfg.num_hidden_layers):
        assert np.array_equal(a.kv_read(layer, 10)[0].view(np.uint32), b.kv_read(layer, 10)[0].view(np.uint32))
    k, v = b.kv_read(0, 3)
    b.kv_write(0, 3, (k + 0.5)[None], v[None])
    assert not np.array_equal(b.forward_token(int(toks[11]), 11), a.forward_token(int(toks[11]), 11))
    with pytest.raises(oracle_mod.OracleError):
        b.kv_write(0, 31, np.zeros((2, cfg.kv_dim()), np.float32), np.zeros((2, cfg.kv_dim()), np.float32))


def test_llama3_rope_table_matches_hf_fixture(oracle_mod):
    """Llama-3 RoPE scaling (no reference counterpart): the oracle's table and
    the library's vvli_host_llama3_inv_freq against Hugging Face's
    _compute_llama3_parameters (tests/golden/llama3_rope.npz, make_rope_golden.py)."""
    from vvli_amd import runtime as R

    data = np.load(GOLDEN / "llama3_rope.npz")
    for name in ("llama32", "llama31"):
        hd, theta, factor, lo, hi, orig = data[name + "_params"]
        ref = data[name]
        args = (int(hd), float(theta), float(factor), float(lo), float(hi), int(orig))
        for got in (oracle_mod.llama3_inv_freq(*args), R.llama3_inv_freq(*args)):
            np.testing.assert_allclose(got, ref, rtol=2e-7, atol=0)
        # Band structure of the closed form: short wavelengths keep the
        # reference frequency, long ones are divided by `factor`.
        base = oracle_mod.llama3_inv_freq(int(hd), float(theta), 1.0, 1.0, 4.0, int(orig))
        wl = 2 * np.pi / base
        assert np.all(ref[wl < orig / hi] == base[wl < orig / hi])
        np.testing.assert_allclose(ref[wl > orig / lo], base[wl > orig / lo] / factor, rtol=1e-6)


def test_llama3_rope_table_rejects_bad_parameters(oracle_mod):
    from vvli_amd import runtime as R
    from vvli_amd._lib import VvliError

    with pytest.raises(VvliError):
        R.llama3_inv_freq(63, 5e5)
    with pytest.raises(VvliError):
        R.llama3_inv_freq(64, 5e5, factor=8.0, low_freq_factor=4.0, high_freq_factor=1.0)
