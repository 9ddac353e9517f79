"""Checkpoint loaders (src/llm.zig:839-1226, src/gguf.zig:234-354) on the CPU.

Pinned without running the reference:
* safetensors files come from independent writers: the ``safetensors``
  package, and HF transformers' ``save_pretrained`` of tiny Llama / Qwen2 /
  Mistral models built from local config objects (no fetch);
* GGUF files come from a byte builder that follows the reference's own parser
  test (src/gguf.zig:356-409) and the published GGUF layout;
* the expected blob places each tensor at the oracle's layout offsets with
  numpy's own conversions (f16 -> f32 by ``astype``, f32 -> bf16 by integer
  round-to-nearest-even), so a wrong name, order, offset or conversion fails.
"""
import json
import struct

import numpy as np
import pytest
import torch

from vvli_amd import _lib
from vvli_amd import config as C
from vvli_amd import loaders as L


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def tensor_list(cfg: C.Config, names: str):
    """(hf or gguf name, slot key, layer, shape) in OwnedModel.assignSlices order."""
    h, kv, inter, v = cfg.hidden_size, cfg.kv_dim(), cfg.intermediate_size, cfg.vocab_size
    hf = names == "hf"
    out = [("model.embed_tokens.weight" if hf else "token_embd.weight", "embed", None, (v, h))]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}." if hf else f"blk.{i}."
        rows = [
            ("input_layernorm.weight", "attn_norm.weight", "input_norm", (h,)),
            ("self_attn.q_proj.weight", "attn_q.weight", "q", (h, h)),
            ("self_attn.q_proj.bias", None, "q_bias", (h,)),
            ("self_attn.k_proj.weight", "attn_k.weight", "k", (kv, h)),
            ("self_attn.k_proj.bias", None, "k_bias", (kv,)),
            ("self_attn.v_proj.weight", "attn_v.weight", "v", (kv, h)),
            ("self_attn.v_proj.bias", None, "v_bias", (kv,)),
            ("self_attn.o_proj.weight", "attn_output.weight", "o", (h, h)),
            ("post_attention_layernorm.weight", "ffn_norm.weight", "post_norm", (h,)),
            ("mlp.gate_proj.weight", "ffn_gate.weight", "gate", (inter, h)),
            ("mlp.up_proj.weight", "ffn_up.weight", "up", (inter, h)),
            ("mlp.down_proj.weight", "ffn_down.weight", "down", (h, inter)),
        ]
        for hn, gn, key, shape in rows:
            if key.endswith("_bias") and not cfg.qkv_bias:
                continue
            out.append((p + (hn if hf else gn), key, i, shape))
    out.append(("model.norm.weight" if hf else "output_norm.weight", "final_norm", None, (h,)))
    if not cfg.tie_word_embeddings:
        out.append(("lm_head.weight" if hf else "output.weight", "lm_head", None, (v, h)))
    return out


def expected_blob(oracle_mod, cfg, tensors: dict, names: str, kind: int) -> np.ndarray:
    """tensors: name -> float32 values (already at the file's precision)."""
    lay = oracle_mod.layout(cfg, kind)
    blob = np.zeros(lay["total"], np.uint16 if kind == C.WEIGHT_BF16 else np.float32)
    for name, key, layer, _shape in tensor_list(cfg, names):
        off = lay[key] if layer is None else lay["layers"][layer][key]
        vals = np.ascontiguousarray(tensors[name], np.float32).reshape(-1)
        blob[off:off + vals.size] = f32_to_bf16_bits(vals) if kind == C.WEIGHT_BF16 else vals
    return blob


def tiny(arch="qwen2", tie=False, bias=True) -> C.Config:
    cfg = C.tiny_test()
    cfg.architecture = arch
    cfg.tie_word_embeddings = tie
    cfg.qkv_bias = bias
    return cfg


# ---------------------------------------------------------------------------
# element conversions
# ---------------------------------------------------------------------------
def test_f16_to_f32_every_bit_pattern():
    lib = _lib.lib()
    bits = np.arange(1 << 16, dtype=np.uint32)
    got = np.array([lib.vvli_host_f16_to_f32(int(b)) for b in bits], np.float32).view(np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan], ref.view(np.uint32)[~nan])
    # NaNs: sign and payload move into the wider mantissa. ctypes widens the
    # returned float to a double, which sets the quiet bit of signalling NaNs,
    # so the quiet bit is masked here; test_gguf_f16_special_values checks the
    # exact bits as they land in the blob.
    nb = bits[nan]
    assert np.array_equal(got[nan] | 0x400000, ((nb & 0x8000) << 16) | 0x7FC00000 | ((nb & 0x3FF) << 13))


# ---------------------------------------------------------------------------
# Config.fromJson edge cases (the reference's four config tests run in
# test_oracle.py through the same parser)
# ---------------------------------------------------------------------------
BASE = {"model_type": "llama", "vocab_size": 32, "hidden_size": 16, "intermediate_size": 32,
        "num_hidden_layers": 2, "num_attention_heads": 4, "max_position_embeddings": 64}


def cfg_err(obj) -> str:
    text = obj if isinstance(obj, str) else json.dumps(obj)
    with pytest.raises(_lib.VvliError) as e:
        C.Config.from_json(text)
    return e.value.name


def test_config_json_defaults_and_token_ids():
    cfg = C.Config.from_json(json.dumps(BASE))
    assert (cfg.num_key_value_heads, cfg.rope_theta, cfg.tie_word_embeddings, cfg.qkv_bias) == (4, 10000.0, False, False)
    assert cfg.rms_norm_eps == np.float32(1e-6) and cfg.rope_layout == C.ROPE_SPLIT_HALF
    assert (cfg.eos_token_id, cfg.pad_token_id) == (0, 0)
    cfg = C.Config.from_json(json.dumps({**BASE, "eos_token_id": [7, 9], "pad_token_id": None, "rope_theta": 500000,
                                         "rms_norm_eps": 1e-5, "num_key_value_heads": 2}))
    assert (cfg.eos_token_id, cfg.pad_token_id, cfg.rope_theta, cfg.num_key_value_heads) == (7, 0, 500000.0, 2)
    assert C.Config.from_json(json.dumps({**BASE, "model_type": "qwen2"})).qkv_bias
    assert not C.Config.from_json(json.dumps({**BASE, "model_type": "qwen2", "attention_bias": False})).qkv_bias
    # Optional fields of the wrong type fall back to their defaults.
    cfg = C.Config.from_json(json.dumps({**BASE, "num_key_value_heads": 2.0, "tie_word_embeddings": 1,
                                         "rope_theta": "x", "eos_token_id": [], "pad_token_id": -1}))
    assert (cfg.num_key_value_heads, cfg.tie_word_embeddings, cfg.rope_theta, cfg.eos_token_id, cfg.pad_token_id) == \
        (4, False, 10000.0, 0, 0)
    # Escapes and unicode in strings, nested values, whitespace.
    text = ' \n{"note": "a\\"b\\u00e9\\ud83d\\ude00", "rope_scaling": {"x": [1, 2.5e-3, null, true]},' + \
        json.dumps(BASE)[1:]
    assert C.Config.from_json(text).vocab_size == 32


def test_config_json_errors():
    assert cfg_err({k: v for k, v in BASE.items() if k != "vocab_size"}) == "MissingJsonField"
    assert cfg_err({k: v for k, v in BASE.items() if k != "model_type"}) == "MissingJsonField"
    assert cfg_err({**BASE, "model_type": 3}) == "MissingJsonField"
    assert cfg_err({**BASE, "model_type": "gpt2"}) == "UnsupportedModelArchitecture"
    assert cfg_err({**BASE, "vocab_size": -1}) == "InvalidConfig"
    assert cfg_err({**BASE, "vocab_size": 32.0}) == "InvalidConfig"
    assert cfg_err({**BASE, "vocab_size": "32"}) == "InvalidConfig"
    assert cfg_err(json.dumps(BASE).replace('"vocab_size": 32', '"vocab_size": 18446744073709551615')) == \
        "InvalidConfig"  # a usize, but wider than the C config's 32-bit field
    assert cfg_err({**BASE, "num_attention_heads": 3}) == "InvalidConfig"  # Config.validate
    assert cfg_err("[1, 2]") == "InvalidConfig"
    for bad in ("", "{", '{"a": 1,}', '{"a": 01}', '{"a": "\\x"}', "{} {}", '{"a": tru}'):
        assert cfg_err(bad) == "InvalidFile", bad


# ---------------------------------------------------------------------------
# safetensors
# ---------------------------------------------------------------------------
def random_tensors(cfg, names, seed, dtype_of=lambda name: torch.float32):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, _key, _layer, shape in tensor_list(cfg, names):
        t = torch.randn(shape, generator=g) * 0.5
        out[name] = t.to(dtype_of(name))
    return out


def as_f32(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


@pytest.mark.parametrize("kind", [C.WEIGHT_F32, C.WEIGHT_BF16])
@pytest.mark.parametrize("file_dtype", ["F32", "BF16", "mixed"])
@pytest.mark.parametrize("arch,tie,bias", [("qwen2", False, True), ("llama", True, False)])
def test_safetensors_blob(oracle_mod, tmp_path, kind, file_dtype, arch, tie, bias):
    from safetensors.torch import save_file

    cfg = tiny(arch, tie, bias)
    pick = {"F32": lambda n: torch.float32, "BF16": lambda n: torch.bfloat16,
            "mixed": lambda n: torch.bfloat16 if sum(map(ord, n)) % 2 else torch.float32}[file_dtype]
    tensors = random_tensors(cfg, "hf", 3, pick)
    tensors["unused.extra"] = torch.zeros(3)  # other entries are ignored
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path))
    seen = []
    blob = L.load_safetensors(cfg, path, kind, progress=lambda d, t, n: seen.append((d, t, n)))
    ref = expected_blob(oracle_mod, cfg, {k: as_f32(v) for k, v in tensors.items()}, "hf", kind)
    assert blob.dtype == ref.dtype and np.array_equal(blob, ref)
    names = [n for n, *_ in tensor_list(cfg, "hf")]
    # weightLoadStepCount: 9 tensors per layer (+3 biases), embed, norm, lm_head if untied.
    assert len(names) == 2 + cfg.num_hidden_layers * (12 if bias else 9) + (0 if tie else 1)
    assert seen == [(0, len(names), "start")] + [(i + 1, len(names), n) for i, n in enumerate(names)]
    # The same image from memory.
    assert np.array_equal(L.safetensors_into_blob(cfg, path.read_bytes(), kind), ref)


def load_err(cfg, data, kind=C.WEIGHT_BF16) -> str:
    with pytest.raises(_lib.VvliError) as e:
        L.safetensors_into_blob(cfg, data, kind)
    return e.value.name


def st_image(header: dict, data: bytes) -> bytes:
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


def test_safetensors_errors(tmp_path):
    from safetensors.torch import save

    cfg = tiny("llama", True, False)
    good = random_tensors(cfg, "hf", 1)
    assert load_err(cfg, save({k: v for k, v in good.items() if k != "model.norm.weight"})) == \
        "MissingSafetensorsTensor"
    wrong_shape = dict(good)
    wrong_shape["model.layers.1.mlp.up_proj.weight"] = torch.zeros(31, 16)
    assert load_err(cfg, save(wrong_shape)) == "InvalidWeight"
    # Same element count in another shape is accepted (the reference checks counts only).
    reshaped = dict(good)
    reshaped["model.layers.1.mlp.up_proj.weight"] = good["model.layers.1.mlp.up_proj.weight"].reshape(16, 32)
    L.safetensors_into_blob(cfg, save(reshaped))
    f16 = dict(good)
    f16["model.embed_tokens.weight"] = good["model.embed_tokens.weight"].half()
    assert load_err(cfg, save(f16)) == "UnsupportedDType"
    img = save(good)
    assert load_err(cfg, img[:7]) == "InvalidWeight"  # shorter than the length prefix
    assert load_err(cfg, img[:-4]) == "InvalidWeight"  # last tensor's data truncated
    assert load_err(cfg, struct.pack("<Q", 1 << 40) + b"{}") == "InvalidWeight"
    assert load_err(cfg, struct.pack("<Q", 3) + b"{x}") == "InvalidFile"
    assert load_err(cfg, st_image([], b"")) == "InvalidWeight"  # header is not an object
    name = "model.embed_tokens.weight"
    n = 24 * 16
    base = {name: {"dtype": "F32", "shape": [24, 16], "data_offsets": [0, 4 * n]}}
    assert load_err(cfg, st_image({**base, name: {**base[name], "data_offsets": [0, 4 * n - 4]}}, bytes(4 * n))) == \
        "InvalidWeight"  # byte length does not match the dtype
    assert load_err(cfg, st_image({**base, name: {**base[name], "data_offsets": [8, 4]}}, bytes(4 * n))) == \
        "InvalidWeight"  # end < start
    assert load_err(cfg, st_image({**base, name: {**base[name], "data_offsets": [-1, 4]}}, bytes(4 * n))) == \
        "InvalidConfig"  # jsonValueUsize on an offset
    assert load_err(cfg, st_image({**base, name: {"shape": [24, 16], "data_offsets": [0, 4 * n]}}, bytes(4 * n))) == \
        "InvalidWeight"
    assert load_err(cfg, st_image({**base, name: {**base[name], "shape": [24, "16"]}}, bytes(4 * n))) == \
        "InvalidWeight"
    moe = C.Config.from_json(json.dumps({**BASE, "num_experts": 4, "num_experts_per_tok": 2}))
    with pytest.raises(_lib.VvliError) as e:
        L.safetensors_into_blob(moe, img, C.WEIGHT_BF16)
    assert e.value.name == "UnsupportedModelArchitecture"
    with pytest.raises(_lib.VvliError) as e:
        L.load_safetensors(cfg, tmp_path / "absent.safetensors")
    assert e.value.name == "InvalidFile"


HF_MODELS = {
    "qwen2": ("Qwen2Config", "Qwen2ForCausalLM", dict(tie_word_embeddings=False)),
    "llama": ("LlamaConfig", "LlamaForCausalLM", dict(tie_word_embeddings=True, attention_bias=False)),
    "mistral": ("MistralConfig", "MistralForCausalLM", dict(tie_word_embeddings=False)),
}


@pytest.mark.parametrize("arch", sorted(HF_MODELS))
@pytest.mark.parametrize("save_dtype", [torch.float32, torch.bfloat16])
def test_hf_save_pretrained_directory(oracle_mod, tmp_path, arch, save_dtype):
    """A directory written by transformers' save_pretrained loads like
    loadOwnedFromDirectory: config.json parsed, every weight at its slot."""
    transformers = pytest.importorskip("transformers")
    cname, mname, extra = HF_MODELS[arch]
    hcfg = getattr(transformers, cname)(vocab_size=40, hidden_size=32, intermediate_size=48, num_hidden_layers=2,
                                        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                                        rope_theta=12345.0, rms_norm_eps=1e-5, eos_token_id=3, pad_token_id=1,
                                        **extra)
    torch.manual_seed(0)
    model = getattr(transformers, mname)(hcfg).to(save_dtype)
    model.save_pretrained(str(tmp_path), safe_serialization=True)
    state = {k: v.float().numpy() for k, v in model.state_dict().items()}
    for kind in (C.WEIGHT_F32, C.WEIGHT_BF16):
        cfg, blob = L.load_directory(tmp_path, kind)
        assert (cfg.architecture, cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
                cfg.num_attention_heads, cfg.num_key_value_heads, cfg.max_position_embeddings) == \
            (arch, 40, 32, 48, 2, 4, 2, 64)
        # transformers 5 nests rope_theta under "rope_parameters"; Config.fromJson
        # reads only the top-level key (src/llm.zig:138), so the default applies.
        assert cfg.rope_theta == 10000.0 and cfg.rms_norm_eps == np.float32(1e-5)
        assert (cfg.eos_token_id, cfg.pad_token_id) == (3, 1)
        assert cfg.qkv_bias == (arch == "qwen2") and cfg.tie_word_embeddings == extra["tie_word_embeddings"]
        assert np.array_equal(blob, expected_blob(oracle_mod, cfg, state, "hf", kind))
    # A config.json with the top-level key (as transformers 4 wrote it) is read.
    conf = json.loads((tmp_path / "config.json").read_text())
    conf["rope_theta"] = conf["rope_parameters"]["rope_theta"]
    (tmp_path / "config.json").write_text(json.dumps(conf))
    assert L.load_directory(tmp_path, C.WEIGHT_BF16)[0].rope_theta == 12345.0


# ---------------------------------------------------------------------------
# GGUF
# ---------------------------------------------------------------------------
U8, I8, U16, I16, U32, I32, F32T, BOOL, STR, ARR, U64, I64, F64 = range(13)
GG_F32, GG_F16, GG_Q8_0, GG_BF16 = 0, 1, 8, 30


class GgufWriter:
    """Little-endian GGUF image builder (the writeString / writeInt helpers of
    src/gguf.zig:411-424 and the layout gguf.parse reads)."""

    def __init__(self, version=3, alignment=None):
        self.version, self.alignment = version, alignment
        self.meta, self.tensors = [], []

    @staticmethod
    def s(text: str) -> bytes:
        b = text.encode()
        return struct.pack("<Q", len(b)) + b

    def kv(self, key, vtype, payload: bytes):
        self.meta.append(self.s(key) + struct.pack("<I", vtype) + payload)
        return self

    def u32(self, key, v): return self.kv(key, U32, struct.pack("<I", v))
    def i32(self, key, v): return self.kv(key, I32, struct.pack("<i", v))
    def f32(self, key, v): return self.kv(key, F32T, struct.pack("<f", v))
    def str_(self, key, v): return self.kv(key, STR, self.s(v))

    def str_array(self, key, items):
        return self.kv(key, ARR, struct.pack("<IQ", STR, len(items)) + b"".join(self.s(i) for i in items))

    def tensor(self, name, dims, ttype, data: bytes, offset=None):
        self.tensors.append([name, list(dims), ttype, data, offset])
        return self

    def build(self, pad_data=True) -> bytes:
        align = self.alignment or 32
        meta = list(self.meta)
        if self.alignment is not None:
            meta.append(self.s("general.alignment") + struct.pack("<II", U32, self.alignment))
        # Data section: each tensor at an aligned offset relative to data start.
        cursor, blobs = 0, []
        for t in self.tensors:
            if t[4] is None:
                cursor = (cursor + align - 1) // align * align
                t[4] = cursor
            blobs.append((t[4], t[3]))
            cursor = max(cursor, t[4] + len(t[3]))
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(meta)) + b"".join(meta)
        for name, dims, ttype, _data, off in self.tensors:
            head += self.s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", ttype, off)
        start = (len(head) + align - 1) // align * align
        out = bytearray(head + bytes(start - len(head)))
        if pad_data:
            out += bytes(cursor)
            for off, data in blobs:
                out[start + off:start + off + len(data)] = data
        return bytes(out)


def gguf_for(cfg, arch="llama", dtype_of=lambda name: GG_F32, seed=0, version=3, alignment=None):
    """A dense model in llama.cpp naming; returns (image, name -> f32 values as stored)."""
    rng = np.random.default_rng(seed)
    w = GgufWriter(version, alignment)
    w.str_("general.architecture", arch)
    w.u32(f"{arch}.block_count", cfg.num_hidden_layers)
    w.u32(f"{arch}.embedding_length", cfg.hidden_size)
    w.u32(f"{arch}.feed_forward_length", cfg.intermediate_size)
    w.u32(f"{arch}.attention.head_count", cfg.num_attention_heads)
    w.u32(f"{arch}.attention.head_count_kv", cfg.num_key_value_heads)
    w.u32(f"{arch}.context_length", cfg.max_position_embeddings)
    w.f32(f"{arch}.rope.freq_base", cfg.rope_theta)
    w.f32(f"{arch}.attention.layer_norm_rms_epsilon", cfg.rms_norm_eps)
    w.str_array("tokenizer.ggml.tokens", [f"t{i}" for i in range(cfg.vocab_size)])
    w.u32("tokenizer.ggml.eos_token_id", cfg.eos_token_id)
    w.i32("tokenizer.ggml.padding_token_id", cfg.pad_token_id)
    values = {}
    for name, _key, _layer, shape in tensor_list(cfg, "gguf"):
        v = (rng.standard_normal(shape) * 0.5).astype(np.float32)
        tt = dtype_of(name)
        if tt == GG_F16:
            v = v.astype(np.float16)
            raw, v = v.tobytes(), v.astype(np.float32)
        elif tt == GG_BF16:
            b = f32_to_bf16_bits(v)
            raw, v = b.tobytes(), bf16_bits_to_f32(b)
        else:
            raw = v.tobytes()
        values[name] = v.reshape(shape)
        w.tensor(name, shape[::-1], tt, raw)  # ggml lists dims fastest-first
    return w, values


def gguf_cfg(tie=True):
    cfg = tiny("llama", tie, False)
    cfg.rope_layout = C.ROPE_INTERLEAVED
    cfg.rms_norm_eps = float(np.float32(1e-5))  # the C config holds f32
    cfg.pad_token_id = 5
    return cfg


@pytest.mark.parametrize("kind", [C.WEIGHT_F32, C.WEIGHT_BF16])
@pytest.mark.parametrize("types", ["f32", "f16", "bf16", "mixed"])
@pytest.mark.parametrize("version,alignment,tie", [(3, None, True), (2, 64, False), (3, 8, True)])
def test_gguf_blob(oracle_mod, tmp_path, kind, types, version, alignment, tie):
    want = gguf_cfg(tie)
    pick = {"f32": lambda n: GG_F32, "f16": lambda n: GG_F16, "bf16": lambda n: GG_BF16,
            "mixed": lambda n: (GG_F32, GG_F16, GG_BF16)[sum(map(ord, n)) % 3]}[types]
    w, values = gguf_for(want, dtype_of=pick, version=version, alignment=alignment)
    img = w.build()
    path = tmp_path / "m.gguf"
    path.write_bytes(img)
    seen = []
    cfg, blob = L.load_gguf(path, kind, progress=lambda d, t, n: seen.append(n))
    assert cfg == want
    assert np.array_equal(blob, expected_blob(oracle_mod, cfg, values, "gguf", kind))
    assert seen == ["start"] + [n for n, *_ in tensor_list(cfg, "gguf")]
    cfg2, blob2 = L.gguf_into_blob(img, kind)
    assert cfg2 == want and np.array_equal(blob2, blob)


def f16_to_f32_bits(h: np.ndarray) -> np.ndarray:
    """binary16 -> binary32 bits: numpy's conversion, NaN payloads shifted over."""
    h = h.astype(np.uint16)
    out = h.view(np.float16).astype(np.float32).view(np.uint32).copy()
    hb = h.astype(np.uint32)
    nan = ((hb & 0x7C00) == 0x7C00) & ((hb & 0x3FF) != 0)
    out[nan] = ((hb[nan] & 0x8000) << 16) | 0x7F800000 | ((hb[nan] & 0x3FF) << 13)
    return out


def test_gguf_f16_special_values():
    """Subnormals, infinities and NaNs (quiet and signalling) in an F16 tensor:
    exact into an f32 blob; into a bf16 blob through f32ToBf16 with no NaN
    special case (src/llm.zig:799-803), so e.g. f16 0x7fff becomes bf16 0x8000."""
    cfg = gguf_cfg()
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8001, 0x0400, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00,
                         0x7C01, 0x7DFF, 0x7E00, 0x7FFF, 0xFC01, 0xFE00, 0xFFFF, 0x3C00, 0x3555], np.uint16)
    n = cfg.vocab_size * cfg.hidden_size
    h = np.resize(specials, n)
    w, _ = gguf_for(cfg)
    w.tensors[0][2] = GG_F16
    w.tensors[0][3] = h.tobytes()
    img = w.build()
    f32_bits = f16_to_f32_bits(h)
    assert f32_bits[np.where(h == 0x7FFF)[0][0]] == 0x7FFFE000
    _, blob = L.gguf_into_blob(img, C.WEIGHT_F32)
    assert np.array_equal(blob[:n].view(np.uint32), f32_bits)
    _, blob = L.gguf_into_blob(img, C.WEIGHT_BF16)
    want = ((f32_bits.astype(np.uint64) + 0x7FFF + ((f32_bits >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(blob[:n], want)
    assert blob[np.where(h == 0x7FFF)[0][0]] == 0x8000


def test_gguf_reference_parser_fixture():
    """The file of src/gguf.zig:356-409: parses (version 3, alignment 32), but
    carries no attention.head_count, so Config.fromGguf stops at MissingJsonField."""
    w = GgufWriter(3)
    w.str_("general.architecture", "llama").u32("llama.block_count", 16).u32("general.alignment", 32)
    w.str_array("tokenizer.ggml.tokens", ["hello", "world"])
    w.tensor("token_embd.weight", [4, 8], GG_F32, b"", offset=0)
    img = w.build(pad_data=False)
    assert len(img) % 32 == 0
    with pytest.raises(_lib.VvliError) as e:
        C.Config.from_gguf(img)
    assert e.value.name == "MissingJsonField" and "llama.attention.head_count" in str(e.value)
    # With the remaining keys the same file yields a config (vocab = 2 token strings).
    for key, v in (("llama.attention.head_count", 2), ("llama.embedding_length", 8),
                   ("llama.feed_forward_length", 16), ("llama.context_length", 32)):
        w.u32(key, v)
    cfg = C.Config.from_gguf(w.build(pad_data=False))
    assert (cfg.vocab_size, cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.rope_theta) == (2, 16, 2, 10000.0)
    assert cfg.rope_layout == C.ROPE_INTERLEAVED and cfg.tie_word_embeddings and not cfg.qkv_bias
    assert cfg.rms_norm_eps == np.float32(1e-6) and (cfg.eos_token_id, cfg.pad_token_id) == (0, 0)


def gguf_err(img, kind=C.WEIGHT_BF16) -> str:
    with pytest.raises(_lib.VvliError) as e:
        L.gguf_into_blob(img, kind)
    return e.value.name


def test_gguf_errors():
    cfg = gguf_cfg()
    w, _ = gguf_for(cfg)
    img = w.build()
    assert gguf_err(b"GGUX" + img[4:]) == "InvalidFile"
    for v in (1, 4):
        assert gguf_err(img[:4] + struct.pack("<I", v) + img[8:]) == "UnsupportedGgufVersion"
    assert gguf_err(img[:20]) == "InvalidFile"  # truncated in the tables
    assert gguf_err(img[:3]) == "InvalidFile"
    # Unknown metadata value type.
    bad = GgufWriter(3).kv("x", 13, b"")
    assert gguf_err(bad.build()) == "UnsupportedMetadataType"
    # Unknown tensor type id; zero and nine dims.
    for dims, tt, name in (([4], 31, "UnsupportedMetadataType"), ([], GG_F32, "InvalidFile"),
                           ([1] * 9, GG_F32, "InvalidFile")):
        w2, _ = gguf_for(cfg)
        w2.tensor("extra", dims, tt, b"")
        assert gguf_err(w2.build()) == name, (dims, tt)
    # general.alignment = 0.
    w2, _ = gguf_for(cfg)
    w2.u32("general.alignment", 0)
    assert gguf_err(w2.build()) == "InvalidFile"
    # Quantised tensor where a weight is needed.
    w2, _ = gguf_for(cfg, dtype_of=lambda n: GG_Q8_0 if n == "blk.1.ffn_up.weight" else GG_F32)
    assert gguf_err(w2.build()) == "UnsupportedDType"
    # Element count mismatch; missing tensor; data past the end of the file.
    w2, _ = gguf_for(cfg)
    w2.tensors[3][1] = [16, 9]  # blk.0.attn_k holds 8 x 16
    assert gguf_err(w2.build()) == "InvalidWeight"
    w2, _ = gguf_for(cfg)
    w2.tensors = [t for t in w2.tensors if t[0] != "output_norm.weight"]
    assert gguf_err(w2.build()) == "MissingSafetensorsTensor"
    assert gguf_err(img[:-8]) == "InvalidWeight"
    # Missing or malformed metadata.
    w2, _ = gguf_for(cfg)
    w2.meta = [m for m in w2.meta if b"tokenizer.ggml.tokens" not in m]
    assert gguf_err(w2.build()) == "MissingJsonField"
    w2, _ = gguf_for(cfg)
    w2.meta = [m for m in w2.meta if b"feed_forward_length" not in m]
    w2.i32("llama.feed_forward_length", -32)  # negative signed integers are not usizes
    assert gguf_err(w2.build()) == "MissingJsonField"
    w2, _ = gguf_for(cfg, arch="gpt2")
    assert gguf_err(w2.build()) == "UnsupportedModelArchitecture"
    # olmoe parses (dense config) but the dense runner rejects it at load.
    w2, _ = gguf_for(cfg, arch="olmoe")
    assert C.Config.from_gguf(w2.build()).architecture == "olmoe"
    assert gguf_err(w2.build()) == "UnsupportedModelArchitecture"
    # A config with q/k/v bias cannot come from GGUF.
    biased = gguf_cfg()
    biased.qkv_bias = True
    blob = np.zeros(biased.storage_element_count(C.WEIGHT_BF16), np.uint16)
    buf = np.frombuffer(img, np.uint8)
    rc = _lib.lib().vvli_host_load_gguf(biased.to_c(C.WEIGHT_BF16), buf.ctypes.data, buf.size, blob.ctypes.data,
                                        blob.size, ctypes_null_progress(), None)
    assert _lib.ERROR_NAMES[rc] == "UnsupportedModelArchitecture"


def ctypes_null_progress():
    import ctypes

    return ctypes.cast(None, _lib.PROGRESS_FN)


def test_gguf_metadata_value_types():
    """Every metadata type is read (and arrays, nested too, are skipped) so that
    the keys after them still parse; usize / f32 lookups accept the integer
    and float types gguf.File.usizeValue / f32Value accept."""
    cfg = gguf_cfg()
    w, _ = gguf_for(cfg)
    extra = GgufWriter()
    extra.kv("a.u8", U8, b"\x01").kv("a.i8", I8, b"\xff").kv("a.u16", U16, b"\x01\x00")
    extra.kv("a.i16", I16, b"\x01\x00").kv("a.bool", BOOL, b"\x01").kv("a.u64", U64, struct.pack("<Q", 9))
    extra.kv("a.i64", I64, struct.pack("<q", -9)).kv("a.f64", F64, struct.pack("<d", 0.5))
    extra.kv("a.nested", ARR, struct.pack("<IQ", ARR, 2) + struct.pack("<IQ", U32, 2) + bytes(8) +
             struct.pack("<IQ", STR, 1) + GgufWriter.s("x"))
    w.meta = extra.meta + w.meta
    # Replace two config keys by other integer / float encodings.
    w.meta = [m for m in w.meta if b"llama.context_length" not in m and b"rope.freq_base" not in m]
    w.kv("llama.context_length", U64, struct.pack("<Q", cfg.max_position_embeddings))
    w.kv("llama.rope.freq_base", F64, struct.pack("<d", 20000.0))
    got = C.Config.from_gguf(w.build())
    assert got.max_position_embeddings == cfg.max_position_embeddings and got.rope_theta == 20000.0
    w.meta = [m for m in w.meta if b"rope.freq_base" not in m]
    w.kv("llama.rope.freq_base", I16, struct.pack("<h", 5000))
    assert C.Config.from_gguf(w.build()).rope_theta == 5000.0


@pytest.mark.parametrize("tie", [True, False])
def test_written_gguf_loads_back_bit_exact(tmp_path, tie):
    """vvli_amd.gguf_write (the benchmark's GGUF workload) read back by the host
    GGUF loader: the same config and the same blob, bit for bit."""
    from vvli_amd import gguf_write
    from vvli_amd import runtime as R

    cfg = tiny("llama", tie, False)
    cfg.rope_layout = C.ROPE_INTERLEAVED
    cfg.rms_norm_eps = float(np.float32(1e-5))
    cfg.rope_theta = float(np.float32(5e5))
    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=3, stddev=0.02)
    path = tmp_path / "m.gguf"
    size = gguf_write.write_dense_gguf(path, cfg, blob)
    assert path.stat().st_size == size
    got_cfg, got = L.load_gguf(path, C.WEIGHT_BF16)
    for f in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "max_position_embeddings", "tie_word_embeddings", "qkv_bias", "rope_layout"):
        assert getattr(got_cfg, f) == getattr(cfg, f), f
    assert got_cfg.rope_theta == cfg.rope_theta and got_cfg.rms_norm_eps == cfg.rms_norm_eps
    np.testing.assert_array_equal(got, blob)
    with pytest.raises(ValueError):
        gguf_write.write_dense_gguf(path, cfg, blob.astype(np.float32))
