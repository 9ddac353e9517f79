"""A dense bf16 blob written out as a GGUF file that the GGUF loaders read
(Config.fromGguf, src/llm.zig:153-193; the container layout of gguf.parse,
src/gguf.zig:234-354; llama.cpp tensor names): how a Llama-shaped model with
random weights becomes the bf16 GGUF workload the benchmark loads.

Metadata: general.architecture, <arch>.block_count / embedding_length /
feed_forward_length / attention.head_count / attention.head_count_kv /
context_length / rope.freq_base / attention.layer_norm_rms_epsilon, and
tokenizer.ggml.tokens (its length is the vocabulary). Tensors are type BF16
(ggml type 30), dimensions listed fastest first, data 32-byte aligned. q / k
are written as they sit in the blob: GGUF models use the interleaved RoPE
pairing, which is what the loaders set (rope_layout 0)."""
from __future__ import annotations

import os
import struct

import numpy as np

from .config import Config, ROPE_INTERLEAVED
from .runtime import dense_slices

_U32, _I32, _F32, _STR, _ARR = 4, 5, 6, 8, 9
_GGML_BF16 = 30
_ALIGN = 32

_NAMES = {"input_norm": "attn_norm", "q": "attn_q", "q_bias": "attn_q", "k": "attn_k", "k_bias": "attn_k",
          "v": "attn_v", "v_bias": "attn_v", "o": "attn_output", "post_norm": "ffn_norm", "gate": "ffn_gate",
          "up": "ffn_up", "down": "ffn_down"}


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def _tensor_shape(cfg: Config, slot: str) -> tuple:
    H, kv, I, V = cfg.hidden_size, cfg.kv_dim(), cfg.intermediate_size, cfg.vocab_size
    return {"embed": (V, H), "lm_head": (V, H), "final_norm": (H,), "input_norm": (H,), "post_norm": (H,),
            "q": (H, H), "q_bias": (H,), "k": (kv, H), "k_bias": (kv,), "v": (kv, H), "v_bias": (kv,),
            "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}[slot]


def _tensor_name(slot: str, layer) -> str:
    if layer is None:
        return {"embed": "token_embd.weight", "final_norm": "output_norm.weight", "lm_head": "output.weight"}[slot]
    return f"blk.{layer}.{_NAMES[slot]}.{'bias' if slot.endswith('_bias') else 'weight'}"


def write_dense_gguf(path: str | os.PathLike, cfg: Config, blob: np.ndarray, arch: str = "llama") -> int:
    """Writes blob (uint16 bf16 bits, the dense layout of cfg) to path; returns
    the file size. The model must use the interleaved RoPE pairing (the one a
    GGUF file implies) and no q/k/v bias (Config.fromGguf sets none)."""
    if blob.dtype != np.uint16:
        raise ValueError("write_dense_gguf takes a bf16 blob (uint16 bits)")
    if cfg.rope_layout != ROPE_INTERLEAVED or cfg.qkv_bias:
        raise ValueError("a GGUF model has interleaved RoPE pairs and no q/k/v bias")
    slices = dense_slices(cfg)
    meta = [
        _s("general.architecture") + struct.pack("<I", _STR) + _s(arch),
        _s(f"{arch}.block_count") + struct.pack("<II", _U32, cfg.num_hidden_layers),
        _s(f"{arch}.embedding_length") + struct.pack("<II", _U32, cfg.hidden_size),
        _s(f"{arch}.feed_forward_length") + struct.pack("<II", _U32, cfg.intermediate_size),
        _s(f"{arch}.attention.head_count") + struct.pack("<II", _U32, cfg.num_attention_heads),
        _s(f"{arch}.attention.head_count_kv") + struct.pack("<II", _U32, cfg.num_key_value_heads),
        _s(f"{arch}.context_length") + struct.pack("<II", _U32, cfg.max_position_embeddings),
        _s(f"{arch}.rope.freq_base") + struct.pack("<If", _F32, cfg.rope_theta),
        _s(f"{arch}.attention.layer_norm_rms_epsilon") + struct.pack("<If", _F32, cfg.rms_norm_eps),
        _s("tokenizer.ggml.tokens") + struct.pack("<IIQ", _ARR, _STR, cfg.vocab_size)
        + b"".join(_s(f"t{i}") for i in range(cfg.vocab_size)),
    ]
    infos, cursor = [], 0
    for slot, layer, off, n in slices:
        shape = _tensor_shape(cfg, slot)
        assert int(np.prod(shape)) == n
        cursor = (cursor + _ALIGN - 1) // _ALIGN * _ALIGN
        infos.append((_tensor_name(slot, layer), shape[::-1], cursor, off, n))
        cursor += 2 * n
    head = b"GGUF" + struct.pack("<IQQ", 3, len(infos), len(meta)) + b"".join(meta)
    for name, dims, data_off, _off, _n in infos:
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", _GGML_BF16, data_off)
    start = (len(head) + _ALIGN - 1) // _ALIGN * _ALIGN
    with open(path, "wb") as f:
        f.write(head + bytes(start - len(head)))
        pos = 0
        for _name, _dims, data_off, off, n in infos:
            if data_off > pos:
                f.write(bytes(data_off - pos))
            f.write(memoryview(blob[off:off + n]).cast("B"))
            pos = data_off + 2 * n
    return start + pos
