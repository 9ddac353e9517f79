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
from vvli_amd._lib import VvliError as VvliErr

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


# ---------------------------------------------------------------------------
# Device-side loading (vvli_gpu_model_create_from_*): the blob written in HBM
# must equal, bit for bit, the blob the host loader builds from the same file.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("kind", [C.WEIGHT_F32, C.WEIGHT_BF16])
def test_device_gguf_blob_equals_host(kind, tmp_path):
    from test_loaders import GG_BF16, GG_F16, GG_F32, gguf_cfg, gguf_for

    want = gguf_cfg(tie=False)
    w, _ = gguf_for(want, dtype_of=lambda n: (GG_F32, GG_F16, GG_BF16)[sum(map(ord, n)) % 3])
    # f16 special values (subnormals, infinities, quiet and signalling NaNs) in the embedding.
    specials = np.array([0x0001, 0x03FF, 0x7C00, 0xFC00, 0x7C01, 0x7E00, 0x7FFF, 0xFFFF, 0x3C00], np.uint16)
    n = want.vocab_size * want.hidden_size
    w.tensors[0][2] = GG_F16
    w.tensors[0][3] = np.resize(specials, n).tobytes()
    path = tmp_path / "m.gguf"
    path.write_bytes(w.build())
    cfg, host = L.load_gguf(path, kind)
    print(f"device gguf kind={kind}", flush=True)
    cfg2, runner = L.device_load_gguf(path, 16, kind)
    with runner:
        assert cfg2 == cfg
        dev = runner.read_weights(0, host.size)
        assert np.array_equal(dev.view(np.uint16 if kind == C.WEIGHT_BF16 else np.uint32),
                              host.view(np.uint16 if kind == C.WEIGHT_BF16 else np.uint32))


@pytest.mark.parametrize("kind", [C.WEIGHT_F32, C.WEIGHT_BF16])
def test_device_safetensors_equals_host(kind, tmp_path):
    from safetensors.torch import save_file
    from test_loaders import random_tensors, tiny

    cfg = tiny("qwen2", False, True)
    tensors = random_tensors(cfg, "hf", 5, lambda n: torch.bfloat16 if sum(map(ord, n)) % 2 else torch.float32)
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path))
    host = L.load_safetensors(cfg, path, kind)
    seen = []
    print(f"device safetensors kind={kind}", flush=True)
    with L.device_load_safetensors(cfg, path, 16, kind, progress=lambda d, t, n: seen.append(n)) as runner:
        assert np.array_equal(runner.read_weights(0, host.size), host)
        assert seen[0] == "start" and seen[-1] == "lm_head.weight"
        with R.Runner(cfg, host, 16) as ref:
            for pos, tok in enumerate([3, 7, 1]):
                assert np.array_equal(runner.forward_token(tok, pos), ref.forward_token(tok, pos))


def test_device_loader_errors(tmp_path):
    from safetensors.torch import save_file
    from test_loaders import random_tensors, tiny

    cfg = tiny("llama", True, False)
    t = random_tensors(cfg, "hf", 1)
    del t["model.norm.weight"]
    path = tmp_path / "model.safetensors"
    save_file(t, str(path))
    with pytest.raises(VvliErr) as e:
        L.device_load_safetensors(cfg, path, 16)
    assert e.value.name == "MissingSafetensorsTensor"
    (tmp_path / "bad.gguf").write_bytes(b"GGUF" + bytes(60))
    with pytest.raises(VvliErr) as e:
        L.device_load_gguf(tmp_path / "bad.gguf", 16)
    assert e.value.name == "UnsupportedGgufVersion"


def test_device_convert_spans_staging_chunks(tmp_path):
    """An f32 embedding of 9000 x 2048 (70 MiB) converted to bf16 on the device
    crosses the 64 MiB staging buffer: every chunk must land at its offset."""
    from safetensors.torch import save_file
    from test_loaders import random_tensors

    cfg = C.Config(vocab_size=9000, hidden_size=2048, intermediate_size=256, num_hidden_layers=1,
                   num_attention_heads=16, num_key_value_heads=4, max_position_embeddings=16, rope_theta=1e4,
                   rms_norm_eps=1e-6, tie_word_embeddings=True, architecture="llama", qkv_bias=False)
    path = tmp_path / "model.safetensors"
    save_file(random_tensors(cfg, "hf", 9), str(path))
    host = L.load_safetensors(cfg, path, C.WEIGHT_BF16)
    print("device safetensors 70 MiB embedding", flush=True)
    with L.device_load_safetensors(cfg, path, 16, C.WEIGHT_BF16) as runner:
        assert np.array_equal(runner.read_weights(0, host.size), host)
