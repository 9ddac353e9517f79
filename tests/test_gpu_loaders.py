"""Models loaded by the checkpoint loaders run on the GPU and match both the
oracle (same blob) and HF transformers' own forward pass of the saved model.

HF side: a tiny Qwen2 / Llama built from a local config object (no fetch),
weights rounded to bf16 and computed in f32 on the CPU; saved with
save_pretrained and read back through load_directory. GGUF side: a tiny
llama-style file (interleaved RoPE) from the byte builder of test_loaders.
Bar: logits within 2e-3 max relative error, as for the forward tests.
"""
import numpy as np
import pytest
import torch

from vvli_amd import config as C
from vvli_amd import loaders as L
from vvli_amd import runtime as R

pytestmark = pytest.mark.gpu

TOL = 2e-3


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


HF = {
    "qwen2": ("Qwen2Config", "Qwen2ForCausalLM", dict(tie_word_embeddings=True)),
    "llama": ("LlamaConfig", "LlamaForCausalLM", dict(tie_word_embeddings=False, attention_bias=False)),
}


@pytest.mark.parametrize("arch", sorted(HF))
def test_hf_directory_runs_like_hf(arch, tmp_path, oracle_mod, host_threads):
    transformers = pytest.importorskip("transformers")
    cname, mname, extra = HF[arch]
    hcfg = getattr(transformers, cname)(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                                        rms_norm_eps=1e-6, **extra)
    torch.manual_seed(0)
    model = getattr(transformers, mname)(hcfg).eval()
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.to(torch.bfloat16).float())  # the values a bf16 blob holds
    model.save_pretrained(str(tmp_path), safe_serialization=True)
    cfg, blob = L.load_directory(tmp_path, C.WEIGHT_BF16)
    tokens = np.random.default_rng(2).integers(0, cfg.vocab_size, size=12)
    with torch.no_grad():
        hf_logits = model(torch.tensor(tokens[None, :], dtype=torch.long)).logits[0].double().numpy()
    orc = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
    print(f"case=hf_{arch} tokens={len(tokens)}", flush=True)
    with R.Runner(cfg, blob, 64) as gpu:
        for pos, tok in enumerate(tokens):
            got = gpu.forward_token(int(tok), pos)
            ref = orc.forward_token(int(tok), pos)
            assert rel_err(got, ref) <= TOL, f"{arch} pos {pos}: vs oracle"
            assert rel_err(got, hf_logits[pos]) <= TOL, f"{arch} pos {pos}: vs HF"


def test_gguf_file_runs_like_oracle(tmp_path, oracle_mod, host_threads):
    from test_loaders import GG_BF16, GG_F16, GG_F32, gguf_for

    want = C.Config(vocab_size=600, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                    num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=128, rope_theta=5e5,
                    rms_norm_eps=float(np.float32(1e-5)), tie_word_embeddings=False, architecture="llama",
                    qkv_bias=False, rope_layout=C.ROPE_INTERLEAVED, eos_token_id=2, pad_token_id=0)
    w, _ = gguf_for(want, dtype_of=lambda n: (GG_F32, GG_F16, GG_BF16)[sum(map(ord, n)) % 3])
    # gguf_for draws N(0, 0.25) weights; scale them down so logits stay O(1).
    for t in w.tensors:
        if not t[0].endswith("norm.weight"):
            dt = {GG_F32: np.float32, GG_F16: np.float16, GG_BF16: np.uint16}[t[2]]
            a = np.frombuffer(t[3], dt)
            if t[2] == GG_BF16:
                a = ((a.astype(np.uint32) << 16).view(np.float32) * 0.125).view(np.uint32) >> 16
                t[3] = a.astype(np.uint16).tobytes()
            else:
                t[3] = (a * dt(0.125)).astype(dt).tobytes()
    path = tmp_path / "m.gguf"
    path.write_bytes(w.build())
    cfg, blob = L.load_gguf(path, C.WEIGHT_BF16)
    assert cfg == want
    orc = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
    tokens = np.random.default_rng(3).integers(0, cfg.vocab_size, size=16)
    print("case=gguf_llama", flush=True)
    with R.Runner(cfg, blob, 64) as gpu:
        for pos, tok in enumerate(tokens):
            e = rel_err(gpu.forward_token(int(tok), pos), orc.forward_token(int(tok), pos))
            assert e <= TOL, f"gguf pos {pos}: {e:.3e}"
