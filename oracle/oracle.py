"""ctypes wrapper of liboracle (vvli_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and bench.py's
CPU-baseline leg, as the source of reference results. The product path never
uses it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, byref, c_float, c_int, c_int64, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libvvli_oracle.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


class OrcConfig(ctypes.Structure):
    _fields_ = [
        ("vocab", c_uint32),
        ("hidden", c_uint32),
        ("inter", c_uint32),
        ("layers", c_uint32),
        ("heads", c_uint32),
        ("kv_heads", c_uint32),
        ("max_pos", c_uint32),
        ("rope_layout", c_uint32),
        ("weight_kind", c_uint32),
        ("tie", c_uint32),
        ("qkv_bias", c_uint32),
        ("rope_theta", c_float),
        ("rms_eps", c_float),
    ]


class OrcLayerOffsets(ctypes.Structure):
    _fields_ = [(n, c_size_t) for n in
                ("input_norm", "q", "q_bias", "k", "k_bias", "v", "v_bias", "o", "post_norm", "gate", "up", "down")]


class OrcMoeConfig(ctypes.Structure):
    _fields_ = [("base", OrcConfig), ("experts", c_uint32), ("top_k", c_uint32), ("qk_norm", c_uint32)]


MOE_SLOTS = ("input_norm", "q", "q_bias", "k", "k_bias", "v", "v_bias", "q_norm", "k_norm", "o", "post_norm", "router",
             "gate_up", "down")


class OrcMoeLayerOffsets(ctypes.Structure):
    _fields_ = [(n, c_size_t) for n in MOE_SLOTS]


class OrcSampling(ctypes.Structure):
    _fields_ = [("temperature", c_float), ("top_p", c_float), ("top_k", c_uint32), ("repeat_penalty", c_float),
                ("repeat_last_n", c_uint32), ("seed", c_uint64)]


class OrcStats(ctypes.Structure):
    _fields_ = [("prompt_tokens", c_uint64), ("generated_tokens", c_uint64), ("prefill_ns", c_int64),
                ("decode_ns", c_int64), ("total_ns", c_int64)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = POINTER
        sig = {
            "orc_bf16_to_f32": (c_float, [c_uint16]),
            "orc_f32_to_bf16": (c_uint16, [c_float]),
            "orc_f16_to_f32": (c_float, [c_uint16]),
            "orc_config_validate": (c_int, [P(OrcConfig)]),
            "orc_parameter_count": (c_size_t, [P(OrcConfig)]),
            "orc_storage_element_count": (c_size_t, [P(OrcConfig)]),
            "orc_layout": (c_size_t, [P(OrcConfig), c_void_p, P(c_size_t), P(c_size_t), P(c_size_t)]),
            "orc_fill_deterministic": (None, [c_void_p, c_size_t, c_uint32]),
            "orc_linear": (None, [c_void_p, c_void_p, c_uint32, c_size_t, c_size_t, c_void_p, c_void_p, c_int]),
            "orc_linear_threaded": (c_int, [c_void_p, c_void_p, c_uint32, c_size_t, c_size_t, c_void_p, c_void_p, c_int,
                                            c_int, c_int]),
            "orc_rmsnorm": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_size_t, c_float, c_int]),
            "orc_rope": (None, [c_void_p, c_size_t, c_size_t, c_size_t, c_float, c_uint32, c_void_p]),
            "orc_llama3_inv_freq": (c_int, [c_uint32, c_float, c_float, c_float, c_float, c_uint32, c_void_p]),
            "orc_softmax": (None, [c_void_p, c_size_t]),
            "orc_attention": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_size_t,
                                     c_void_p, c_int]),
            "orc_silu_mul": (None, [c_void_p, c_void_p, c_void_p, c_size_t]),
            "orc_add": (None, [c_void_p, c_void_p, c_void_p, c_size_t]),
            "orc_argmax": (c_size_t, [c_void_p, c_size_t]),
            "orc_dot_f32": (c_float, [c_void_p, c_void_p, c_size_t, c_int]),
            "orc_dot_bf16": (c_float, [c_void_p, c_void_p, c_size_t, c_int]),
            "orc_runner_create": (c_int, [P(OrcConfig), c_void_p, c_size_t, c_uint32, c_int, c_int, P(c_void_p)]),
            "orc_runner_destroy": (None, [c_void_p]),
            "orc_kv_clear": (None, [c_void_p]),
            "orc_set_rope_table": (c_int, [c_void_p, c_void_p, c_uint32]),
            "orc_forward_token": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
            "orc_prefill": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_void_p]),
            "orc_forward_embedding": (c_int, [c_void_p, c_void_p, c_uint32, c_void_p, c_void_p]),
            "orc_kv_read": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
            "orc_kv_write": (c_int, [c_void_p, c_uint32, c_uint32, c_uint32, c_void_p, c_void_p]),
            "orc_generate_greedy": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_int64, c_void_p, P(c_uint32),
                                            P(OrcStats)]),
            "orc_moe_layout": (c_size_t, [P(OrcMoeConfig), c_void_p, P(c_size_t), P(c_size_t), P(c_size_t)]),
            "orc_moe_rmsnorm": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_size_t, c_float]),
            "orc_moe_route": (None, [c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]),
            "orc_moe_experts": (c_int, [c_void_p, c_void_p, c_uint32, c_size_t, c_size_t, c_void_p, c_size_t,
                                        c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_int, c_int, c_int]),
            "orc_matmul_blocked": (None, [c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_int]),
            "orc_moe_runner_create": (c_int, [P(OrcMoeConfig), c_void_p, c_size_t, c_uint32, c_int, c_int,
                                              P(c_void_p)]),
            "orc_moe_runner_destroy": (None, [c_void_p]),
            "orc_moe_forward_token": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p]),
            "orc_moe_kv_read": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
            "orc_splitmix64_next": (c_uint64, [P(c_uint64)]),
            "orc_prng_seed": (None, [c_void_p, c_uint64]),
            "orc_prng_next": (c_uint64, [c_void_p]),
            "orc_prng_float": (c_float, [c_void_p]),
            "orc_build_candidates": (c_size_t, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, P(OrcSampling)]),
            "orc_prepare_probabilities": (c_size_t, [c_void_p, c_void_p, c_size_t, P(OrcSampling)]),
            "orc_sample_candidate": (c_uint32, [c_void_p, c_void_p, c_size_t, c_float]),
            "orc_sampler_next": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, P(OrcSampling),
                                         c_void_p, P(c_uint32)]),
            "orc_generate_sampled": (c_int, [c_void_p, c_size_t, c_void_p, c_uint32, c_uint32, c_int64,
                                             P(OrcSampling), c_void_p, P(c_uint32)]),
            "orc_adjusted_logit": (c_float, [c_float, c_uint16, c_float]),
            "orc_greedy_with_penalties": (c_uint32, [c_void_p, c_void_p, c_size_t, c_float]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else c_void_p(a.ctypes.data)


def orc_config(cfg, weight_kind: int) -> OrcConfig:
    """From a vvli_amd.config.Config (or anything with the same attributes)."""
    c = OrcConfig()
    c.vocab = cfg.vocab_size
    c.hidden = cfg.hidden_size
    c.inter = cfg.intermediate_size
    c.layers = cfg.num_hidden_layers
    c.heads = cfg.num_attention_heads
    c.kv_heads = cfg.num_key_value_heads
    c.max_pos = cfg.max_position_embeddings
    c.rope_layout = cfg.rope_layout
    c.weight_kind = weight_kind
    c.tie = int(cfg.tie_word_embeddings)
    c.qkv_bias = int(cfg.qkv_bias)
    c.rope_theta = cfg.rope_theta
    c.rms_eps = cfg.rms_norm_eps
    return c


# ---- ops ----
def bf16_to_f32(bits: int) -> float:
    return lib().orc_bf16_to_f32(bits)


def f32_to_bf16(v: float) -> int:
    return lib().orc_f32_to_bf16(v)


def linear(w: np.ndarray, x: np.ndarray, bias: np.ndarray | None = None, lanes: int = 16) -> np.ndarray:
    rows, cols = w.shape
    kind = 1 if w.dtype == np.uint16 else 0
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(rows, dtype=np.float32)
    lib().orc_linear(_p(out), _p(w), kind, rows, cols, _p(x), _p(bias), lanes)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, lanes: int = 16) -> np.ndarray:
    kind = 1 if w.dtype == np.uint16 else 0
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_rmsnorm(_p(out), _p(x), _p(np.ascontiguousarray(w)), kind, x.size, eps, lanes)
    return out


def llama3_inv_freq(head_dim: int, theta: float, factor: float, low_freq_factor: float, high_freq_factor: float,
                    original_max_pos: int) -> np.ndarray:
    out = np.zeros(head_dim // 2, dtype=np.float32)
    _check(lib().orc_llama3_inv_freq(head_dim, theta, factor, low_freq_factor, high_freq_factor, original_max_pos,
                                     _p(out)))
    return out


def rope(values: np.ndarray, heads: int, head_dim: int, pos: int, theta: float, layout: int,
         inv_freq: np.ndarray | None = None) -> np.ndarray:
    v = np.array(values, dtype=np.float32, copy=True)
    t = None if inv_freq is None else np.ascontiguousarray(inv_freq, dtype=np.float32)
    lib().orc_rope(_p(v), heads, head_dim, pos, theta, layout, _p(t))
    return v


def softmax(values: np.ndarray) -> np.ndarray:
    v = np.array(values, dtype=np.float32, copy=True)
    lib().orc_softmax(_p(v), v.size)
    return v


def attention(q, keys, values, heads, kv_heads, head_dim, pos, lanes=16) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    keys = np.ascontiguousarray(keys, dtype=np.float32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    scores = np.zeros(pos + 1, dtype=np.float32)
    lib().orc_attention(_p(out), _p(q), _p(keys), _p(values), heads, kv_heads, head_dim, pos, _p(scores), lanes)
    return out


def silu_mul(g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.zeros_like(g)
    lib().orc_silu_mul(_p(out), _p(g), _p(u), g.size)
    return out


def argmax(logits) -> int:
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().orc_argmax(_p(a), a.size))


def storage_element_count(cfg, weight_kind: int) -> int:
    c = orc_config(cfg, weight_kind)
    return int(lib().orc_storage_element_count(byref(c)))


def parameter_count(cfg) -> int:
    c = orc_config(cfg, 1)
    return int(lib().orc_parameter_count(byref(c)))


def layout(cfg, weight_kind: int) -> dict:
    c = orc_config(cfg, weight_kind)
    arr = (OrcLayerOffsets * cfg.num_hidden_layers)()
    e, fn, lm = c_size_t(), c_size_t(), c_size_t()
    total = lib().orc_layout(byref(c), arr, byref(e), byref(fn), byref(lm))
    none = (1 << 64) - 1
    layers = [{k: (None if getattr(a, k) == none else getattr(a, k)) for k, _ in OrcLayerOffsets._fields_} for a in arr]
    return {"embed": e.value, "final_norm": fn.value, "lm_head": None if lm.value == none else lm.value,
            "layers": layers, "total": int(total)}


def fill_deterministic(n: int, weight_kind: int) -> np.ndarray:
    blob = np.zeros(n, dtype=np.uint16 if weight_kind == 1 else np.float32)
    lib().orc_fill_deterministic(_p(blob), n, weight_kind)
    return blob


class OracleError(RuntimeError):
    def __init__(self, rc: int):
        self.rc = rc
        super().__init__(f"oracle rc={rc}")


def _check(rc: int) -> None:
    if rc:
        raise OracleError(rc)


class OracleRunner:
    """CPU restatement of llm.Runner; borrows ``blob`` (kept alive here)."""

    def __init__(self, cfg, blob: np.ndarray, max_seq_len: int, threads: int = 0, lanes: int = 16):
        self.cfg = cfg
        self.blob = np.ascontiguousarray(blob)
        kind = 1 if self.blob.dtype == np.uint16 else 0
        self._c = orc_config(cfg, kind)
        h = c_void_p()
        _check(lib().orc_runner_create(byref(self._c), _p(self.blob), self.blob.size, max_seq_len, threads, lanes,
                                       byref(h)))
        self._h = h
        self.logits = np.zeros(cfg.vocab_size, dtype=np.float32)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().orc_runner_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward_token(self, token: int, pos: int, want_hidden: bool = False):
        hidden = (np.zeros((self.cfg.num_hidden_layers, self.cfg.hidden_size), dtype=np.float32)
                  if want_hidden else None)
        _check(lib().orc_forward_token(self._h, token, pos, _p(self.logits), _p(hidden)))
        return (self.logits.copy(), hidden) if want_hidden else self.logits.copy()

    def forward_embedding(self, emb: np.ndarray, pos: int, want_hidden: bool = False):
        emb = np.ascontiguousarray(emb, dtype=np.float32)
        hidden = (np.zeros((self.cfg.num_hidden_layers, self.cfg.hidden_size), dtype=np.float32)
                  if want_hidden else None)
        _check(lib().orc_forward_embedding(self._h, _p(emb), pos, _p(self.logits), _p(hidden)))
        return (self.logits.copy(), hidden) if want_hidden else self.logits.copy()

    def prefill(self, tokens, start_pos: int = 0) -> np.ndarray:
        """The prompt loop with its loops interchanged (orc_prefill): same KV
        rows and last logits as one forward_token per token."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        _check(lib().orc_prefill(self._h, _p(toks), toks.size, start_pos, _p(self.logits)))
        return self.logits.copy()

    def kv_read(self, layer: int, pos: int):
        kv = self.cfg.kv_dim() if hasattr(self.cfg, "kv_dim") else None
        k = np.zeros(kv, dtype=np.float32)
        v = np.zeros(kv, dtype=np.float32)
        _check(lib().orc_kv_read(self._h, layer, pos, _p(k), _p(v)))
        return k, v

    def kv_write(self, layer: int, pos: int, k: np.ndarray, v: np.ndarray):
        """Overwrite cache rows pos .. pos + len(k) - 1 of one layer ([n, kv] f32 each)."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        if k.shape != v.shape or k.ndim != 2:
            raise ValueError("k and v must both be [n, kv]")
        _check(lib().orc_kv_write(self._h, layer, pos, k.shape[0], _p(k), _p(v)))

    def kv_clear(self):
        lib().orc_kv_clear(self._h)

    def set_rope_table(self, inv_freq):
        t = None if inv_freq is None else np.ascontiguousarray(inv_freq, dtype=np.float32)
        _check(lib().orc_set_rope_table(self._h, _p(t), 0 if t is None else t.size))

    def generate_sampled(self, prompt, max_new: int, opts, eos: int | None = None):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(1, max_new), dtype=np.uint32)
        n = c_uint32()
        c = orc_sampling(opts)
        _check(lib().orc_generate_sampled(self._h, self.cfg.vocab_size, _p(p), p.size, max_new,
                                          -1 if eos is None else eos, byref(c), _p(out), byref(n)))
        return out[: n.value].copy()

    def generate_greedy(self, prompt, max_new: int, eos: int | None = None):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(1, max_new), dtype=np.uint32)
        n = c_uint32()
        st = OrcStats()
        _check(lib().orc_generate_greedy(self._h, _p(p), p.size, max_new, -1 if eos is None else eos, _p(out),
                                         byref(n), byref(st)))
        return out[: n.value].copy(), st


def orc_sampling(opts) -> OrcSampling:
    return OrcSampling(opts.temperature, opts.top_p, opts.top_k, opts.repeat_penalty, opts.repeat_last_n, opts.seed)


def prng_seed(seed: int) -> np.ndarray:
    st = np.zeros(4, dtype=np.uint64)
    lib().orc_prng_seed(_p(st), seed)
    return st


def sampler_next(logits, prompt, generated, opts, prng_state: np.ndarray) -> int:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    p = np.ascontiguousarray(prompt, dtype=np.uint32)
    g = np.ascontiguousarray(generated, dtype=np.uint32)
    tok = c_uint32()
    c = orc_sampling(opts)
    _check(lib().orc_sampler_next(_p(lg), lg.size, _p(p), p.size, _p(g), g.size, byref(c), _p(prng_state),
                                  byref(tok)))
    return tok.value


def orc_moe_config(cfg, weight_kind: int) -> OrcMoeConfig:
    return OrcMoeConfig(orc_config(cfg, weight_kind), cfg.num_experts, cfg.num_experts_per_token, int(cfg.qk_norm))


def moe_layout(cfg, weight_kind: int) -> dict:
    c = orc_moe_config(cfg, weight_kind)
    arr = (OrcMoeLayerOffsets * cfg.num_hidden_layers)()
    e, fn, lm = c_size_t(), c_size_t(), c_size_t()
    total = lib().orc_moe_layout(byref(c), arr, byref(e), byref(fn), byref(lm))
    none = (1 << 64) - 1
    layers = [{k: (None if getattr(a, k) == none else getattr(a, k)) for k in MOE_SLOTS} for a in arr]
    return {"embed": e.value, "final_norm": fn.value, "lm_head": None if lm.value == none else lm.value,
            "layers": layers, "total": int(total)}


def moe_route(logits: np.ndarray, top_k: int):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(top_k, dtype=np.uint32)
    w = np.zeros(top_k, dtype=np.float32)
    lib().orc_moe_route(_p(lg), lg.size, top_k, _p(idx), _p(w))
    return idx, w


def moe_experts(blob: np.ndarray, kind: int, gate_up: int, down: int, x: np.ndarray, hidden: int, inter: int,
                experts: int, idx: np.ndarray, weights: np.ndarray, matmul: bool, lanes: int = 16,
                threads: int = 1) -> np.ndarray:
    """The routed experts' weighted sum of one layer (orc_moe_experts): each
    product as linearInto (matmul False, the MoE runner's path) or as
    tensor.zig's matmul (matmul True)."""
    out = np.zeros(hidden, dtype=np.float32)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    ii = np.ascontiguousarray(idx, dtype=np.uint32)
    ww = np.ascontiguousarray(weights, dtype=np.float32)
    _check(lib().orc_moe_experts(_p(out), _p(blob), kind, gate_up, down, _p(xx), hidden, inter, experts, ii.size,
                                 _p(ii), _p(ww), lanes, threads, 1 if matmul else 0))
    return out


def matmul_blocked(a: np.ndarray, b: np.ndarray, lanes: int = 16) -> np.ndarray:
    """src/tensor.zig matmulBlocked: a [m][k] . b [k][n], f32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.zeros((a.shape[0], b.shape[1]), dtype=np.float32)
    lib().orc_matmul_blocked(_p(out), _p(a), a.shape[0], a.shape[1], _p(b), b.shape[1], lanes)
    return out


class OracleMoeRunner:
    """CPU restatement of the MoE (OLMoE-form) token step; borrows ``blob``."""

    def __init__(self, cfg, blob: np.ndarray, max_seq_len: int, threads: int = 0, lanes: int = 16):
        self.cfg = cfg
        self.blob = np.ascontiguousarray(blob)
        kind = 1 if self.blob.dtype == np.uint16 else 0
        self._c = orc_moe_config(cfg, kind)
        h = c_void_p()
        _check(lib().orc_moe_runner_create(byref(self._c), _p(self.blob), self.blob.size, max_seq_len, threads, lanes,
                                           byref(h)))
        self._h = h
        self.logits = np.zeros(cfg.vocab_size, dtype=np.float32)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().orc_moe_runner_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward_token(self, token: int, pos: int, want_hidden: bool = False):
        L = self.cfg.num_hidden_layers
        hidden = np.zeros((L, self.cfg.hidden_size), dtype=np.float32) if want_hidden else None
        experts = np.zeros((L, self.cfg.num_experts_per_token), dtype=np.uint32) if want_hidden else None
        _check(lib().orc_moe_forward_token(self._h, token, pos, _p(self.logits), _p(hidden), _p(experts)))
        return (self.logits.copy(), hidden, experts) if want_hidden else self.logits.copy()

    def kv_read(self, layer: int, pos: int):
        kv = self.cfg.kv_dim()
        k = np.zeros(kv, dtype=np.float32)
        v = np.zeros(kv, dtype=np.float32)
        _check(lib().orc_moe_kv_read(self._h, layer, pos, _p(k), _p(v)))
        return k, v

    def generate_greedy(self, prompt, max_new: int):
        """The generator loop (src/generator.zig:243-293) over this step: prompt
        token by token, then the argmax of each step is emitted and forwarded."""
        pos, logits = 0, None
        for t in prompt:
            logits = self.forward_token(int(t), pos)
            pos += 1
        out = []
        for i in range(max_new):
            tok = int(lib().orc_argmax(_p(logits), logits.size))
            out.append(tok)
            logits = self.forward_token(tok, pos)
            pos += 1
        return np.array(out, dtype=np.uint32)


def cpu_count() -> int:
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
