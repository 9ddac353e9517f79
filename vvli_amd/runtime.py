"""Python host over the C ABI, named after VVLI's runner API.

``Runner`` mirrors ``llm.Runner`` (src/llm.zig:688-776): ``forward_token``,
``forward_embedding`` and ``argmax``; ``generate_greedy_measured`` mirrors
``generator.generateGreedyMeasured`` (src/generator.zig:177-293). Every call
goes through libvvli_gpu.so; nothing here computes model math.
"""
from __future__ import annotations

import ctypes
import dataclasses
from ctypes import byref, c_uint32, c_void_p

import numpy as np

from . import _lib
from .config import WEIGHT_BF16, WEIGHT_F32, Config

_DTYPE = {WEIGHT_BF16: np.uint16, WEIGHT_F32: np.float32}


def _ptr(a: np.ndarray | None) -> c_void_p | None:
    return None if a is None else c_void_p(a.ctypes.data)


def empty_blob(cfg: Config, weight_kind: int = WEIGHT_BF16) -> np.ndarray:
    n = cfg.storage_element_count(weight_kind)
    return np.empty(n, dtype=_DTYPE[weight_kind])


def synthetic_blob(cfg: Config, weight_kind: int = WEIGHT_BF16, seed: int = 0, stddev: float = 0.02,
                   threads: int = 0) -> np.ndarray:
    """Seeded N(0, stddev) weights, RMSNorm weights 1 (vvli_host_fill_synthetic)."""
    blob = empty_blob(cfg, weight_kind)
    c = cfg.to_c(weight_kind)
    _lib.check(_lib.lib().vvli_host_fill_synthetic(byref(c), seed, stddev, _ptr(blob), blob.size, threads))
    return blob


def deterministic_blob(cfg: Config, weight_kind: int = WEIGHT_F32) -> np.ndarray:
    """OwnedModel.fillDeterministicForTesting (src/llm.zig:466-477)."""
    blob = empty_blob(cfg, weight_kind)
    _lib.lib().vvli_host_fill_deterministic(_ptr(blob), blob.size, weight_kind)
    return blob


def llama3_inv_freq(head_dim: int, theta: float, factor: float = 32.0, low_freq_factor: float = 1.0,
                    high_freq_factor: float = 4.0, original_max_pos: int = 8192) -> np.ndarray:
    """Llama-3 RoPE frequencies for Runner.set_rope_table (vvli_host_llama3_inv_freq).
    Defaults: Llama-3.2's rope_scaling."""
    out = np.zeros(head_dim // 2, dtype=np.float32)
    _lib.check(_lib.lib().vvli_host_llama3_inv_freq(head_dim, theta, factor, low_freq_factor, high_freq_factor,
                                                     original_max_pos, _ptr(out)))
    return out


def dense_slices(cfg: Config, weight_kind: int = WEIGHT_BF16) -> list:
    """(slot, layer or None, element offset, element count) of every slice of
    the dense blob, in vvli_gpu_storage_element_count's layout (assignSlices,
    src/llm.zig:488-522: embed; per layer input_norm, q, (q_bias), k,
    (k_bias), v, (v_bias), o, post_norm, gate, up, down; final_norm; lm_head
    unless tied; each slice 64-byte aligned)."""
    ea = 64 // (2 if weight_kind == WEIGHT_BF16 else 4)
    H, kv, I = cfg.hidden_size, cfg.kv_dim(), cfg.intermediate_size
    out, cur = [], 0

    def take(slot, layer, n):
        nonlocal cur
        cur = (cur + ea - 1) // ea * ea
        out.append((slot, layer, cur, n))
        cur += n

    take("embed", None, cfg.vocab_size * H)
    for l in range(cfg.num_hidden_layers):
        for slot, n in [("input_norm", H), ("q", H * H), ("q_bias", H if cfg.qkv_bias else None), ("k", kv * H),
                        ("k_bias", kv if cfg.qkv_bias else None), ("v", kv * H),
                        ("v_bias", kv if cfg.qkv_bias else None), ("o", H * H), ("post_norm", H),
                        ("gate", I * H), ("up", I * H), ("down", H * I)]:
            if n is not None:
                take(slot, l, n)
    take("final_norm", None, H)
    if not cfg.tie_word_embeddings:
        take("lm_head", None, cfg.vocab_size * H)
    return out


def moe_slice_offset(cfg: Config, layer: int, slot: str, weight_kind: int = WEIGHT_BF16) -> int:
    """Element offset of one slice of the MoE blob (vvli_gpu_moe_storage_element_count's
    layout: per layer input_norm, q, (q_bias), k, (k_bias), v, (v_bias), (q_norm,
    k_norm), o, post_norm, router, gate_up, down; 64-byte aligned)."""
    ea = 64 // (2 if weight_kind == WEIGHT_BF16 else 4)
    H, kv, I, E = cfg.hidden_size, cfg.kv_dim(), cfg.intermediate_size, cfg.num_experts
    cur = 0

    def take(n):
        nonlocal cur
        cur = (cur + ea - 1) // ea * ea
        at = cur
        cur += n
        return at

    take(cfg.vocab_size * H)
    for l in range(cfg.num_hidden_layers):
        sizes = [("input_norm", H), ("q", H * H), ("q_bias", H if cfg.qkv_bias else None), ("k", kv * H),
                 ("k_bias", kv if cfg.qkv_bias else None), ("v", kv * H), ("v_bias", kv if cfg.qkv_bias else None),
                 ("q_norm", H if cfg.qk_norm else None), ("k_norm", kv if cfg.qk_norm else None), ("o", H * H),
                 ("post_norm", H), ("router", E * H), ("gate_up", E * 2 * I * H), ("down", E * H * I)]
        for name, n in sizes:
            if n is None:
                continue
            at = take(n)
            if l == layer and name == slot:
                return at
    raise KeyError(slot)


def argmax(logits: np.ndarray) -> int:
    """llm.argmax (src/llm.zig:778-789): first index of the strict maximum."""
    best, bv = 0, logits[0]
    for i in range(1, len(logits)):
        if logits[i] > bv:
            best, bv = i, logits[i]
    return best


@dataclasses.dataclass
class Stats:
    """generator.Stats (src/generator.zig:25-43)."""

    prompt_tokens: int
    generated_tokens: int
    prefill_nanoseconds: int
    decode_nanoseconds: int
    total_nanoseconds: int

    def decode_tokens_per_second(self) -> float:
        return _tps(self.generated_tokens, self.decode_nanoseconds)

    def prefill_tokens_per_second(self) -> float:
        return _tps(self.prompt_tokens, self.prefill_nanoseconds)

    def total_tokens_per_second(self) -> float:
        return _tps(self.prompt_tokens + self.generated_tokens, self.total_nanoseconds)


def _tps(tokens: int, ns: int) -> float:
    # tokensPerSecond, src/generator.zig:326-330
    return 0.0 if tokens == 0 or ns <= 0 else tokens * 1e9 / ns


class Runner:
    """Device-resident model + KV cache + scratch on the current HIP device.

    Owns one ``vvli_gpu_model`` handle (weights, f32 KV cache of
    ``max_seq_len`` positions, activations). The host blob is copied to the
    device by the constructor and may be dropped afterwards.
    """

    def __init__(self, cfg: Config, blob: np.ndarray, max_seq_len: int, weight_kind: int | None = None):
        if weight_kind is None:
            weight_kind = WEIGHT_BF16 if blob.dtype == np.uint16 else WEIGHT_F32
        if blob.dtype != _DTYPE[weight_kind]:
            raise TypeError("blob dtype does not match weight_kind")
        self.cfg = cfg
        self.weight_kind = weight_kind
        self.max_seq_len = max_seq_len
        self._c = cfg.to_c(weight_kind)
        handle = c_void_p()
        blob = np.ascontiguousarray(blob)
        _lib.check(self._create(byref(self._c), max_seq_len, _ptr(blob), blob.size, byref(handle)))
        self._h = handle
        self._path = "auto"
        self.logits = np.zeros(cfg.vocab_size, dtype=np.float32)

    @staticmethod
    def _create(*args):
        # llm.Runner: dense decoders only; MoE configs are rejected like OwnedModel.init.
        return _lib.lib().vvli_gpu_model_create(*args)

    @classmethod
    def from_handle(cls, cfg: Config, handle: c_void_p, max_seq_len: int, weight_kind: int) -> "Runner":
        """Wraps a model handle created by another entry point (the device loaders)."""
        r = cls.__new__(cls)
        r.cfg, r.weight_kind, r.max_seq_len = cfg, weight_kind, max_seq_len
        r._c = cfg.to_c(weight_kind)
        r._h = handle
        r._path = "auto"
        r.logits = np.zeros(cfg.vocab_size, dtype=np.float32)
        return r

    def read_weights(self, offset: int, n: int) -> np.ndarray:
        """vvli_gpu_read_weights: n blob elements from offset (blob dtype)."""
        out = np.empty(n, dtype=_DTYPE[self.weight_kind])
        _lib.check(_lib.lib().vvli_gpu_read_weights(self._h, offset, n, _ptr(out)))
        return out

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.check(_lib.lib().vvli_gpu_model_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- llm.Runner ----
    def forward_token(self, token_id: int, position: int) -> np.ndarray:
        """Runner.forwardToken (src/llm.zig:702-709); returns the logits."""
        am = c_uint32()
        _lib.check(_lib.lib().vvli_gpu_forward_token(self._h, token_id, position, _ptr(self.logits), byref(am)))
        self.last_argmax = am.value
        return self.logits

    def forward_token_view(self, token_id: int, position: int) -> np.ndarray:
        """Runner.forwardToken with its borrowed-slice return (src/llm.zig:729):
        a read-only array over the library's pinned logits, overwritten by the
        next forward_token_view call (with resident steps, by the next call
        that returns logits) and invalid once the runner is closed."""
        view = c_void_p()
        am = c_uint32()
        _lib.check(_lib.lib().vvli_gpu_forward_token_view(self._h, token_id, position, byref(view), byref(am)))
        self.last_argmax = am.value
        buf = (ctypes.c_float * self.cfg.vocab_size).from_address(view.value)
        out = np.frombuffer(buf, dtype=np.float32)
        out.flags.writeable = False
        return out

    def forward_token_argmax(self, token_id: int, position: int) -> int:
        am = c_uint32()
        _lib.check(_lib.lib().vvli_gpu_forward_token(self._h, token_id, position, None, byref(am)))
        return am.value

    def forward_embedding(self, embedding: np.ndarray, position: int) -> np.ndarray:
        """Runner.forwardEmbedding (src/llm.zig:711-718)."""
        emb = np.ascontiguousarray(embedding, dtype=np.float32)
        if emb.size != self.cfg.hidden_size:
            raise _lib.VvliError(2, "embedding length != hidden_size")
        am = c_uint32()
        _lib.check(_lib.lib().vvli_gpu_forward_embedding(self._h, _ptr(emb), position, _ptr(self.logits), byref(am)))
        self.last_argmax = am.value
        return self.logits

    def forward_token_debug(self, token_id: int, position: int) -> tuple[np.ndarray, np.ndarray]:
        """forwardToken plus the residual stream after every layer ([layers, hidden])."""
        hidden = np.zeros((self.cfg.num_hidden_layers, self.cfg.hidden_size), dtype=np.float32)
        _lib.check(_lib.lib().vvli_gpu_forward_token_debug(self._h, token_id, position, _ptr(self.logits), _ptr(hidden)))
        return self.logits.copy(), hidden

    def kv_read(self, layer: int, position: int) -> tuple[np.ndarray, np.ndarray]:
        kv = self.cfg.kv_dim()
        k = np.zeros(kv, dtype=np.float32)
        v = np.zeros(kv, dtype=np.float32)
        _lib.check(_lib.lib().vvli_gpu_kv_read(self._h, layer, position, _ptr(k), _ptr(v)))
        return k, v

    def kv_clear(self) -> None:
        _lib.check(_lib.lib().vvli_gpu_kv_clear(self._h))

    def set_rope_table(self, inv_freq: np.ndarray | None) -> None:
        if inv_freq is None:
            _lib.check(_lib.lib().vvli_gpu_set_rope_table(self._h, None, 0))
        else:
            t = np.ascontiguousarray(inv_freq, dtype=np.float32)
            _lib.check(_lib.lib().vvli_gpu_set_rope_table(self._h, _ptr(t), t.size))

    def persistent_available(self) -> bool:
        """True when this model can run the persistent one-launch step (the
        default decode path then)."""
        try:
            self.set_decode_path("persistent")
        except _lib.VvliError:
            return False
        finally:
            self.set_decode_path(self._path)
        return True

    def last_launch_ms(self) -> float:
        """Device time (HIP events) of the last persistent launch: the decode
        launch of generate_greedy_measured, or a prefill / token step."""
        ms = ctypes.c_float()
        _lib.check(_lib.lib().vvli_gpu_last_launch_time(self._h, ctypes.byref(ms)))
        return float(ms.value)

    def set_resident(self, linger_us: int) -> None:
        """Resident single steps: forward_token calls on the persistent path
        hand their (token, position) to a launch that stays running for up to
        linger_us of idle time (0 turns it off). Same results as separate
        launches; other work on the GPU waits while such a launch idles."""
        _lib.check(_lib.lib().vvli_gpu_set_resident(self._h, linger_us))

    def set_decode_path(self, path: str) -> None:
        """'auto', 'graph' (per-kernel HIP graph) or 'persistent' (one launch per step)."""
        _lib.check(_lib.lib().vvli_gpu_set_decode_path(self._h, {"auto": 0, "graph": 1, "persistent": 2}[path]))
        self._path = path

    def set_prefill_path(self, path: str) -> None:
        """'auto', 'loop' (one token step per prompt token) or 'batched' (GEMM prefill)."""
        _lib.check(_lib.lib().vvli_gpu_set_prefill_path(self._h, {"auto": 0, "loop": 1, "batched": 2}[path]))

    def prefill(self, tokens, start_pos: int = 0) -> tuple[np.ndarray, int]:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        am = c_uint32()
        _lib.check(_lib.lib().vvli_gpu_prefill(self._h, _ptr(toks), toks.size, start_pos, _ptr(self.logits), byref(am)))
        return self.logits, am.value

    # ---- generator ----
    def generate(self, prompt, max_new_tokens: int, sampling: "Sampling", eos_token_id: int | None = None,
                 batched_prefill: bool = False) -> tuple[np.ndarray, Stats]:
        """generateGreedyMeasured with Options (src/generator.zig:221-293): sampling on the device."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(1, max_new_tokens), dtype=np.uint32)
        n = c_uint32()
        st = _lib.CStats()
        c = sampling.to_c()
        eos = -1 if eos_token_id is None else int(eos_token_id)
        _lib.check(_lib.lib().vvli_gpu_generate(self._h, _ptr(p), p.size, max_new_tokens, eos,
                                                1 if batched_prefill else 0, byref(c), _ptr(out), byref(n),
                                                byref(st)))
        stats = Stats(st.prompt_tokens, st.generated_tokens, st.prefill_ns, st.decode_ns, st.total_ns)
        return out[: n.value].copy(), stats

    def generate_greedy_measured(self, prompt, max_new_tokens: int, eos_token_id: int | None = None,
                                 batched_prefill: bool = False) -> tuple[np.ndarray, Stats]:
        """generateGreedyMeasured (src/generator.zig:177-293), greedy sampler."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(1, max_new_tokens), dtype=np.uint32)
        n = c_uint32()
        st = _lib.CStats()
        eos = -1 if eos_token_id is None else int(eos_token_id)
        flags = 1 if batched_prefill else 0
        _lib.check(_lib.lib().vvli_gpu_generate_greedy(self._h, _ptr(p), p.size, max_new_tokens, eos, flags, _ptr(out),
                                                       byref(n), byref(st)))
        stats = Stats(st.prompt_tokens, st.generated_tokens, st.prefill_ns, st.decode_ns, st.total_ns)
        return out[: n.value].copy(), stats


class MoeRunner(Runner):
    """Token step of a mixture-of-experts decoder (OLMoE form) through
    vvli_gpu_moe_model_create; same methods as Runner. No reference
    counterpart: the reference runner rejects MoE configs (src/llm.zig:426)."""

    @staticmethod
    def _create(*args):
        return _lib.lib().vvli_gpu_moe_model_create(*args)


@dataclasses.dataclass
class Sampling:
    """generator.Options (src/generator.zig:14-23): the sampler's settings."""

    temperature: float = 0.8
    top_p: float = 0.95
    top_k: int = 40
    repeat_penalty: float = 1.10
    repeat_last_n: int = 64
    seed: int = 0

    def to_c(self) -> _lib.CSampling:
        return _lib.CSampling(self.temperature, self.top_p, self.top_k, self.repeat_penalty, self.repeat_last_n,
                              self.seed)


def prng_seed(seed: int) -> np.ndarray:
    """DefaultPrng.init(seed) as Sampler.init calls it (seed 0 mapped first)."""
    st = np.zeros(4, dtype=np.uint64)
    _lib.lib().vvli_gpu_prng_seed(seed, _ptr(st))
    return st


def sampler_next(logits: np.ndarray, prompt, generated, opts: Sampling, prng_state: np.ndarray) -> int:
    """Sampler.next (src/generator.zig:93-120) on the device; advances prng_state in place."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    p = np.ascontiguousarray(prompt, dtype=np.uint32)
    g = np.ascontiguousarray(generated, dtype=np.uint32)
    assert prng_state.dtype == np.uint64 and prng_state.size == 4 and prng_state.flags.c_contiguous
    tok = c_uint32()
    c = opts.to_c()
    _lib.check(_lib.lib().vvli_gpu_sampler_next(_ptr(lg), lg.size, _ptr(p) if p.size else None, p.size,
                                                _ptr(g) if g.size else None, g.size, byref(c), _ptr(prng_state),
                                                byref(tok)))
    return tok.value


def sampler_trace(logits: np.ndarray, opts: Sampling, prng_state: np.ndarray):
    """vvli_gpu_test_sampler_trace: the whole-vocabulary sampler's token and, in
    candidate order, its candidates' ids, probabilities and running f32 sums."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    assert prng_state.dtype == np.uint64 and prng_state.size == 4 and prng_state.flags.c_contiguous
    ids = np.zeros(lg.size, np.uint32)
    probs = np.zeros(lg.size, np.float32)
    sums = np.zeros(lg.size, np.float32)
    tok, count = c_uint32(), c_uint32()
    c = opts.to_c()
    _lib.check(_lib.lib().vvli_gpu_test_sampler_trace(_ptr(lg), lg.size, byref(c), _ptr(prng_state), byref(tok),
                                                      _ptr(ids), _ptr(probs), _ptr(sums), byref(count)))
    n = count.value
    return tok.value, ids[:n], probs[:n], sums[:n]


def linear(dW: int, dX: int, dY: int, M: int, N: int, K: int, dBias: int | None = None, stream: int | None = None) -> None:
    """vvli_gpu_linear on raw device pointers (e.g. torch ``tensor.data_ptr()``)."""
    _lib.check(_lib.lib().vvli_gpu_linear(c_void_p(dW), c_void_p(dX), None if dBias is None else c_void_p(dBias),
                                          c_void_p(dY), M, N, K, None if stream is None else c_void_p(stream)))


def linear_noalloc(dW: int, dX: int, dY: int, M: int, N: int, K: int, dBias: int | None = None,
                   stream: int | None = None) -> None:
    """vvli_gpu_linear_noalloc: the same op with its scratch in a static device
    array (no allocation; at most VVLI_LINEAR_NOALLOC_SCRATCH_BYTES of split planes)."""
    _lib.check(_lib.lib().vvli_gpu_linear_noalloc(c_void_p(dW), c_void_p(dX), None if dBias is None else c_void_p(dBias),
                                                  c_void_p(dY), M, N, K, None if stream is None else c_void_p(stream)))
