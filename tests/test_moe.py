"""Mixture-of-experts (OLMoE form) on the CPU: the oracle's MoE step against
HF transformers' OlmoeForCausalLM golden fixture, routing special cases, and
the MoE blob layout shared by the library and the oracle.

The reference has no MoE forward pass (src/llm.zig:218-223,426 reject it); the
semantics are HF OLMoE's (QK-norm over the full q / k, router softmax in f32,
top-k without renormalisation, experts summed in ascending id).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from vvli_amd import _lib
from vvli_amd import config as C
from vvli_amd import runtime as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "olmoe_tiny.npz"


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


def fixture():
    z = np.load(GOLDEN)
    conf = json.loads(bytes(z["config"]).decode())
    cfg = C.Config(architecture="olmoe", vocab_size=conf["vocab_size"], hidden_size=conf["hidden_size"],
                   intermediate_size=conf["intermediate_size"], num_hidden_layers=conf["num_hidden_layers"],
                   num_attention_heads=conf["num_attention_heads"], num_key_value_heads=conf["num_key_value_heads"],
                   max_position_embeddings=conf["max_position_embeddings"], rope_theta=conf["rope_theta"],
                   rms_norm_eps=float(np.float32(conf["rms_norm_eps"])), tie_word_embeddings=False, qkv_bias=False,
                   rope_layout=C.ROPE_SPLIT_HALF, num_experts=conf["num_experts"],
                   num_experts_per_token=conf["num_experts_per_tok"], qk_norm=True)
    return z, cfg


def blob_from_hf(oracle_mod, cfg, z, swap_gate_up=False, reverse_experts=False):
    """Places HF OLMoE tensors at the MoE layout's offsets (bf16 blob)."""
    lay = oracle_mod.moe_layout(cfg, C.WEIGHT_BF16)
    blob = np.zeros(lay["total"], np.uint16)

    def put(off, name, transform=None):
        a = z["w/" + name]
        if transform is not None:
            a = transform(a)
        blob[off:off + a.size] = a.reshape(-1)

    put(lay["embed"], "model.embed_tokens.weight")
    I = cfg.intermediate_size
    for i, L in enumerate(lay["layers"]):
        p = f"model.layers.{i}."
        put(L["input_norm"], p + "input_layernorm.weight")
        put(L["q"], p + "self_attn.q_proj.weight")
        put(L["k"], p + "self_attn.k_proj.weight")
        put(L["v"], p + "self_attn.v_proj.weight")
        put(L["q_norm"], p + "self_attn.q_norm.weight")
        put(L["k_norm"], p + "self_attn.k_norm.weight")
        put(L["o"], p + "self_attn.o_proj.weight")
        put(L["post_norm"], p + "post_attention_layernorm.weight")
        put(L["router"], p + "mlp.gate.weight")
        gu = (lambda a: np.concatenate([a[:, I:], a[:, :I]], axis=1)) if swap_gate_up else None
        put(L["gate_up"], p + "mlp.experts.gate_up_proj", gu)
        put(L["down"], p + "mlp.experts.down_proj", (lambda a: a[::-1]) if reverse_experts else None)
    put(lay["final_norm"], "model.norm.weight")
    put(lay["lm_head"], "lm_head.weight")
    return blob


def run_oracle(oracle_mod, cfg, blob, tokens):
    orc = oracle_mod.OracleMoeRunner(cfg, blob, 32, threads=2)
    out = [orc.forward_token(int(t), pos, want_hidden=True) for pos, t in enumerate(tokens)]
    return out


def test_oracle_matches_hf_olmoe_fixture(oracle_mod):
    z, cfg = fixture()
    blob = blob_from_hf(oracle_mod, cfg, z)
    out = run_oracle(oracle_mod, cfg, blob, z["tokens"])
    for pos, (logits, hidden, experts) in enumerate(out):
        assert rel_err(logits, z["logits"][pos]) <= 2e-5, f"pos {pos}"
        assert rel_err(hidden[0], z["hidden"][pos, 0]) <= 2e-5, f"pos {pos} layer 0"
        np.testing.assert_array_equal(experts, z["experts"][pos])  # same experts, same (probability) order


@pytest.mark.parametrize("mistake", ["swap_gate_up", "reverse_experts"])
def test_fixture_detects_planted_mistakes(oracle_mod, mistake):
    """A wrong gate/up order or a wrong expert indexing in the blob must fail
    the comparison the real layout passes."""
    z, cfg = fixture()
    blob = blob_from_hf(oracle_mod, cfg, z, **{mistake: True})
    out = run_oracle(oracle_mod, cfg, blob, z["tokens"])
    assert max(rel_err(lg, z["logits"][p]) for p, (lg, _, _) in enumerate(out)) > 1e-2


def test_route_special_cases(oracle_mod):
    # Closed form: softmax of the logits, largest k, no renormalisation.
    lg = np.array([0.5, 2.0, -1.0, 2.0, 1.0, 0.0], np.float32)
    idx, w = oracle_mod.moe_route(lg, 3)
    p = np.exp(lg.astype(np.float64) - lg.max())
    p /= p.sum()
    assert list(idx) == [1, 3, 4]  # tie between 1 and 3: the lower id first
    np.testing.assert_allclose(w, p[[1, 3, 4]], rtol=1e-6)
    assert w.sum() < 1.0
    idx, w = oracle_mod.moe_route(lg, 6)
    assert list(idx) == [1, 3, 4, 0, 5, 2]
    np.testing.assert_allclose(w.sum(), 1.0, rtol=1e-6)
    idx, w = oracle_mod.moe_route(np.zeros(8, np.float32), 2)
    assert list(idx) == [0, 1] and np.allclose(w, 0.125)


@pytest.mark.parametrize("qkv_bias,qk_norm,tie", [(False, True, False), (True, True, True), (False, False, False)])
def test_moe_layout_library_matches_oracle(oracle_mod, qkv_bias, qk_norm, tie):
    cfg = C.Config(architecture="olmoe", vocab_size=100, hidden_size=64, intermediate_size=48, num_hidden_layers=3,
                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=32, rope_theta=1e4,
                   rms_norm_eps=1e-5, tie_word_embeddings=tie, qkv_bias=qkv_bias, num_experts=6,
                   num_experts_per_token=2, qk_norm=qk_norm)
    lay = oracle_mod.moe_layout(cfg, C.WEIGHT_BF16)
    assert cfg.storage_element_count(C.WEIGHT_BF16) == lay["total"]
    assert cfg.storage_element_count(C.WEIGHT_F32) == oracle_mod.moe_layout(cfg, C.WEIGHT_F32)["total"]
    # Every slice 64-byte aligned, in order, none overlapping.
    offs = [lay["embed"]] + [v for L in lay["layers"] for v in L.values() if v is not None] + [lay["final_norm"]]
    if lay["lm_head"] is not None:
        offs.append(lay["lm_head"])
    assert all(o % 32 == 0 for o in offs) and offs == sorted(offs) and len(set(offs)) == len(offs)
    # The library's synthetic filler writes 1.0 exactly at the oracle's norm slices.
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=3)
    one = np.uint16(0x3F80)
    H, kv = cfg.hidden_size, cfg.kv_dim()
    for L in lay["layers"]:
        for key, n in (("input_norm", H), ("post_norm", H), ("q_norm", H), ("k_norm", kv)):
            if L[key] is not None:
                assert np.all(blob[L[key]:L[key] + n] == one), key
        for key in ("router", "gate_up", "down", "q"):
            assert np.count_nonzero(blob[L[key]:L[key] + 64] == one) < 8, key
    assert np.all(blob[lay["final_norm"]:lay["final_norm"] + H] == one)


def test_moe_runner_rejects_what_it_cannot_run():
    _, cfg = fixture()
    with pytest.raises(_lib.VvliError) as e:  # the dense runner rejects MoE, like OwnedModel.init
        R.Runner(cfg, np.zeros(16, np.uint16), 16)
    assert e.value.name == "UnsupportedModelArchitecture"
    with pytest.raises(_lib.VvliError) as e:  # MoE kernels are bf16-only
        R.MoeRunner(cfg, np.zeros(16, np.float32), 16)
    assert e.value.name == "UnsupportedDType"
    dense = C.tiny_test()
    with pytest.raises(_lib.VvliError) as e:
        R.MoeRunner(dense, np.zeros(16, np.uint16), 16)
    assert e.value.name == "InvalidConfig"


def test_moe_slice_offsets_match_oracle(oracle_mod):
    for cfg in (C.olmoe_1b_7b(), fixture()[1]):
        lay = oracle_mod.moe_layout(cfg, C.WEIGHT_BF16)
        for l in range(cfg.num_hidden_layers):
            for k, v in lay["layers"][l].items():
                if v is not None:
                    assert R.moe_slice_offset(cfg, l, k) == v, (l, k)


def test_tensor_matmul_restatement(oracle_mod):
    """src/tensor.zig matmulBlocked restated: the reference's known answer
    (src/tensor.zig:793-812) and, at the shape of its "no-scratch and
    transposed scratch paths agree" test (:814-846: m 3, k lanes * 4 + 3,
    n lanes * 4 + 5, the panel, vector and scalar column paths), agreement
    with an f64 product within that test's 1e-5, for 4-, 8- and 16-lane hosts."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert np.array_equal(oracle_mod.matmul_blocked(a, b), np.array([[58, 64], [139, 154]], np.float32))
    for lanes in (4, 8, 16):
        m, k, n = 3, lanes * 4 + 3, lanes * 4 + 5
        a = ((np.arange(m * k) % 11) - 5).astype(np.float32).reshape(m, k) * np.float32(0.125)
        b = (((np.arange(k * n) * 3) % 13) - 6).astype(np.float32).reshape(k, n) * np.float32(0.0625)
        got = oracle_mod.matmul_blocked(a, b, lanes)
        ref = a.astype(np.float64) @ b.astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-5, f"lanes {lanes}"
        # A planted mistake (one column of b dropped from a panel) must fail.
        b2 = b.copy()
        b2[:, 1] = 0
        assert np.max(np.abs(oracle_mod.matmul_blocked(a, b2, lanes) - ref)) > 1e-3


@pytest.mark.parametrize("shape", ["fixture", "olmoe-1b-7b-experts"])
def test_moe_experts_tensor_matmul_composition(shape, oracle_mod):
    """The MoE oracle's routed-expert sum (each expert's gate/up and down as
    linearInto, the runner's path) against the same composition with every
    product as the reference's tensor.zig matmul (src/tensor.zig:297-325,
    683-733: the row x times the expert matrix transposed to f32): both
    within 1e-5 of an f64 evaluation and of each other -- the two differ
    only in the f32 summation order of the dot products. Shapes: the HF
    OLMoE fixture's layer 0 (hidden 64, 8 experts of 32, top 2) and an
    OLMoE-1B-7B-shaped expert layer (hidden 2048, experts of 1024, top 8 --
    the per-token expert work of OLMoE-1B-7B -- out of 16 experts instead of
    64, to keep the blob small)."""
    if shape == "fixture":
        z, cfg = fixture()
        blob = blob_from_hf(oracle_mod, cfg, z)
    else:
        cfg = C.olmoe_1b_7b()
        cfg = C.Config(**{**cfg.__dict__, "num_hidden_layers": 1, "vocab_size": 64, "num_experts": 16})
        blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=5, stddev=0.02)
    lay = oracle_mod.moe_layout(cfg, C.WEIGHT_BF16)
    L = lay["layers"][0]
    H, I, E, K = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts, cfg.num_experts_per_token
    rng = np.random.default_rng(3)
    x = rng.standard_normal(H).astype(np.float32)
    idx, w = oracle_mod.moe_route(rng.standard_normal(E).astype(np.float32), K)
    lin = oracle_mod.moe_experts(blob, C.WEIGHT_BF16, L["gate_up"], L["down"], x, H, I, E, idx, w, matmul=False)
    mm = oracle_mod.moe_experts(blob, C.WEIGHT_BF16, L["gate_up"], L["down"], x, H, I, E, idx, w, matmul=True)
    # f64 evaluation of the same composition.
    def f64(off, n):  # bf16 bits of the blob slice -> f64
        return (blob[off:off + n].astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)

    ref = np.zeros(H)
    for e in sorted(int(i) for i in idx):
        gu = f64(L["gate_up"] + e * 2 * I * H, 2 * I * H).reshape(2 * I, H) @ x
        act = gu[:I] / (1 + np.exp(-gu[:I])) * gu[I:]
        out = f64(L["down"] + e * H * I, H * I).reshape(H, I) @ act
        ref += out * float(w[list(idx).index(e)])
    assert rel_err(lin, ref) <= 1e-5 and rel_err(mm, ref) <= 1e-5
    assert rel_err(lin, mm) <= 1e-5
    # A planted mistake (gate and up swapped in one expert) must fail.
    e0 = int(idx[0])
    g0 = L["gate_up"] + e0 * 2 * I * H
    gate = blob[g0:g0 + I * H].copy()
    blob[g0:g0 + I * H] = blob[g0 + I * H:g0 + 2 * I * H]
    blob[g0 + I * H:g0 + 2 * I * H] = gate
    mm_bad = oracle_mod.moe_experts(blob, C.WEIGHT_BF16, L["gate_up"], L["down"], x, H, I, E, idx, w, matmul=True)
    assert rel_err(mm_bad, ref) > 1e-2
