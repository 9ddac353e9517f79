"""Model shape contract: a Python mirror of VVLI's ``llm.Config``.

Fields and defaults follow ``Config`` (src/llm.zig:77-97); the derived sizes
follow ``headDim`` / ``kvDim`` / ``kvGroupSize`` (src/llm.zig:229-239). The
named constructors are the decoder shapes the benchmarks and parity tests run.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from . import _lib

ARCH = {"llama": 0, "mistral": 1, "olmoe": 2, "qwen2": 3}
ROPE_INTERLEAVED, ROPE_SPLIT_HALF = 0, 1
WEIGHT_F32, WEIGHT_BF16 = 0, 1


@dataclasses.dataclass
class Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    max_position_embeddings: int
    rope_theta: float
    rms_norm_eps: float
    tie_word_embeddings: bool
    architecture: str = "qwen2"  # src/llm.zig:78 default
    qkv_bias: bool = True  # src/llm.zig:94 default
    rope_layout: int = ROPE_SPLIT_HALF  # src/llm.zig:89 default
    num_experts: int = 0
    num_experts_per_token: int = 0
    qk_norm: bool = False
    eos_token_id: int = 0
    pad_token_id: int = 0

    # ---- derived sizes (src/llm.zig:229-239) ----
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim()

    def kv_group_size(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    # ---- C ABI ----
    def to_c(self, weight_kind: int = WEIGHT_BF16) -> _lib.CConfig:
        c = _lib.CConfig()
        c.abi_version = _lib.ABI_VERSION
        c.arch = ARCH[self.architecture]
        c.vocab = self.vocab_size
        c.hidden = self.hidden_size
        c.inter = self.intermediate_size
        c.layers = self.num_hidden_layers
        c.heads = self.num_attention_heads
        c.kv_heads = self.num_key_value_heads
        c.max_pos = self.max_position_embeddings
        c.rope_layout = self.rope_layout
        c.weight_kind = weight_kind
        c.num_experts = self.num_experts
        c.experts_per_tok = self.num_experts_per_token
        c.rope_theta = self.rope_theta
        c.rms_eps = self.rms_norm_eps
        c.tie = int(self.tie_word_embeddings)
        c.qkv_bias = int(self.qkv_bias)
        c.qk_norm = int(self.qk_norm)
        c.eos_token_id = self.eos_token_id
        c.pad_token_id = self.pad_token_id
        return c

    def validate(self) -> None:
        """Config.validate (src/llm.zig:195-216), run by the library."""
        _lib.check(_lib.lib().vvli_gpu_config_validate(ctypes.byref(self.to_c())))

    def parameter_count(self) -> int:
        return int(_lib.lib().vvli_gpu_parameter_count(ctypes.byref(self.to_c())))

    def storage_element_count(self, weight_kind: int = WEIGHT_BF16) -> int:
        """Blob elements: the dense layout (storageElementCount, src/llm.zig:814-837),
        or the MoE layout of vvli_gpu_moe_storage_element_count for MoE configs."""
        fn = (_lib.lib().vvli_gpu_moe_storage_element_count if self.num_experts
              else _lib.lib().vvli_gpu_storage_element_count)
        return int(fn(ctypes.byref(self.to_c(weight_kind))))

    @classmethod
    def from_c(cls, c: _lib.CConfig) -> "Config":
        """The inverse of to_c (weight_kind is not part of Config)."""
        names = {v: k for k, v in ARCH.items()}
        return cls(
            architecture=names[c.arch],
            vocab_size=c.vocab,
            hidden_size=c.hidden,
            intermediate_size=c.inter,
            num_hidden_layers=c.layers,
            num_attention_heads=c.heads,
            num_key_value_heads=c.kv_heads,
            max_position_embeddings=c.max_pos,
            rope_layout=c.rope_layout,
            num_experts=c.num_experts,
            num_experts_per_token=c.experts_per_tok,
            rope_theta=c.rope_theta,
            rms_norm_eps=c.rms_eps,
            tie_word_embeddings=bool(c.tie),
            qkv_bias=bool(c.qkv_bias),
            qk_norm=bool(c.qk_norm),
            eos_token_id=c.eos_token_id,
            pad_token_id=c.pad_token_id,
        )

    @classmethod
    def from_json(cls, text: str | bytes) -> "Config":
        """Config.fromJson (src/llm.zig:98-145): HF config.json keys, parsed by
        vvli_host_config_from_json."""
        raw = text.encode() if isinstance(text, str) else bytes(text)
        c = _lib.CConfig()
        _lib.check(_lib.lib().vvli_host_config_from_json(raw, len(raw), WEIGHT_BF16, ctypes.byref(c)))
        return cls.from_c(c)

    @classmethod
    def from_gguf(cls, data) -> "Config":
        """Config.fromGguf (src/llm.zig:153-193) over a whole GGUF image (bytes,
        bytearray, numpy array or anything exposing the buffer protocol)."""
        buf = np.frombuffer(data, dtype=np.uint8)
        c = _lib.CConfig()
        _lib.check(_lib.lib().vvli_host_config_from_gguf(ctypes.c_void_p(buf.ctypes.data), buf.size, WEIGHT_BF16,
                                                         ctypes.byref(c)))
        return cls.from_c(c)


# ---------------------------------------------------------------------------
# Named shapes.
# ---------------------------------------------------------------------------
def tiny_test() -> Config:
    """The reference's tiny runner test (src/llm.zig:1743-1782)."""
    return Config(
        vocab_size=24,
        hidden_size=16,
        intermediate_size=32,
        num_hidden_layers=2,
        num_attention_heads=4,
        num_key_value_heads=2,
        max_position_embeddings=16,
        rope_theta=10_000.0,
        rms_norm_eps=0.000001,
        tie_word_embeddings=True,
        eos_token_id=2,
        pad_token_id=0,
    )


def qwen25_05b() -> Config:
    """Qwen2.5-0.5B: 24 layers, hidden 896, 14/2 heads, inter 4864, vocab 151936, tied, qkv bias."""
    return Config(
        architecture="qwen2",
        vocab_size=151936,
        hidden_size=896,
        intermediate_size=4864,
        num_hidden_layers=24,
        num_attention_heads=14,
        num_key_value_heads=2,
        max_position_embeddings=32768,
        rope_theta=1_000_000.0,
        rms_norm_eps=1e-6,
        tie_word_embeddings=True,
        qkv_bias=True,
        rope_layout=ROPE_SPLIT_HALF,
        eos_token_id=151645,
        pad_token_id=151654,
    )


def llama32_1b() -> Config:
    """Llama-3.2-1B as read from a GGUF (Config.fromGguf, src/llm.zig:153-193):
    interleaved RoPE, no qkv bias, tied (no output.weight)."""
    return Config(
        architecture="llama",
        vocab_size=128256,
        hidden_size=2048,
        intermediate_size=8192,
        num_hidden_layers=16,
        num_attention_heads=32,
        num_key_value_heads=8,
        max_position_embeddings=131072,
        rope_theta=500_000.0,
        rms_norm_eps=1e-5,
        tie_word_embeddings=True,
        qkv_bias=False,
        rope_layout=ROPE_INTERLEAVED,
        eos_token_id=128009,
        pad_token_id=128004,
    )


def qwen25_7b() -> Config:
    """Qwen2.5-7B: 28 layers, hidden 3584, 28/4 heads, hd 128, inter 18944, untied, qkv bias."""
    return Config(
        architecture="qwen2",
        vocab_size=152064,
        hidden_size=3584,
        intermediate_size=18944,
        num_hidden_layers=28,
        num_attention_heads=28,
        num_key_value_heads=4,
        max_position_embeddings=32768,
        rope_theta=1_000_000.0,
        rms_norm_eps=1e-6,
        tie_word_embeddings=False,
        qkv_bias=True,
        rope_layout=ROPE_SPLIT_HALF,
        eos_token_id=151645,
        pad_token_id=151643,
    )


def olmoe_1b_7b() -> Config:
    """OLMoE-1B-7B shape: 16 layers, hidden 2048, 16/16 heads (hd 128), 64
    experts x inter 1024, top-8, QK-norm, vocab 50304, untied."""
    return Config(
        architecture="olmoe",
        vocab_size=50304,
        hidden_size=2048,
        intermediate_size=1024,
        num_hidden_layers=16,
        num_attention_heads=16,
        num_key_value_heads=16,
        max_position_embeddings=4096,
        rope_theta=10_000.0,
        rms_norm_eps=1e-5,
        tie_word_embeddings=False,
        qkv_bias=False,
        rope_layout=ROPE_SPLIT_HALF,
        num_experts=64,
        num_experts_per_token=8,
        qk_norm=True,
        eos_token_id=50279,
        pad_token_id=1,
    )


NAMED = {
    "tiny": tiny_test,
    "qwen2.5-0.5b": qwen25_05b,
    "llama-3.2-1b": llama32_1b,
    "qwen2.5-7b": qwen25_7b,
    "olmoe-1b-7b": olmoe_1b_7b,
}
