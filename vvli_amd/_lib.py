"""ctypes binding of libvvli_gpu.so (include/vvli_gpu.h, include/vvli_host.h).

The library is built in-tree (make -C vvli_amd/csrc). There is no fallback: if the shared object is missing the
import of any runtime object raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint8, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).with_name("libvvli_gpu.so")
ABI_VERSION = 1

# Return codes of include/vvli_gpu.h mapped to the reference's error names
# (src/llm.zig:17-27, src/generator.zig:8-12, src/gguf.zig:7-12).
ERROR_NAMES = {
    1: "InvalidConfig",
    2: "InvalidWeight",
    3: "InvalidToken",
    4: "ContextFull",
    5: "UnsupportedDType",
    6: "UnsupportedModelArchitecture",
    7: "OutOfMemory",
    8: "HipRuntime",
    9: "MissingJsonField",
    10: "EmptyPrompt",
    11: "MissingSafetensorsTensor",
    12: "InvalidFile",
    13: "UnsupportedGgufVersion",
    14: "OutputTooSmall",
    15: "InvalidSamplingOptions",
    16: "UnsupportedMetadataType",
    100: "NullArgument",
}


class VvliError(RuntimeError):
    """A non-zero return code; ``name`` is the reference error it stands for."""

    def __init__(self, rc: int, message: str):
        self.rc = rc
        self.name = ERROR_NAMES.get(rc, f"Error{rc}")
        super().__init__(f"{self.name} (rc={rc}): {message}")


class CConfig(ctypes.Structure):
    _fields_ = [
        ("abi_version", c_uint32),
        ("arch", c_uint32),
        ("vocab", c_uint32),
        ("hidden", c_uint32),
        ("inter", c_uint32),
        ("layers", c_uint32),
        ("heads", c_uint32),
        ("kv_heads", c_uint32),
        ("max_pos", c_uint32),
        ("rope_layout", c_uint32),
        ("weight_kind", c_uint32),
        ("num_experts", c_uint32),
        ("experts_per_tok", c_uint32),
        ("rope_theta", c_float),
        ("rms_eps", c_float),
        ("tie", c_uint8),
        ("qkv_bias", c_uint8),
        ("qk_norm", c_uint8),
        ("_pad", c_uint8),
        ("eos_token_id", c_uint32),
        ("pad_token_id", c_uint32),
    ]


class CStats(ctypes.Structure):
    _fields_ = [
        ("prompt_tokens", c_uint64),
        ("generated_tokens", c_uint64),
        ("prefill_ns", c_int64),
        ("decode_ns", c_int64),
        ("total_ns", c_int64),
    ]


class CSampling(ctypes.Structure):
    _fields_ = [
        ("temperature", c_float),
        ("top_p", c_float),
        ("top_k", c_uint32),
        ("repeat_penalty", c_float),
        ("repeat_last_n", c_uint32),
        ("seed", c_uint64),
    ]


# void (*)(void* user, size_t completed, size_t total, const char* name)
PROGRESS_FN = ctypes.CFUNCTYPE(None, c_void_p, c_size_t, c_size_t, c_char_p)

# name -> (restype, argtypes): every symbol the two headers declare.
PROTOTYPES = {
    "vvli_gpu_abi_version": (c_uint32, []),
    "vvli_gpu_last_error": (c_char_p, []),
    "vvli_gpu_config_validate": (c_int, [POINTER(CConfig)]),
    "vvli_gpu_parameter_count": (c_uint64, [POINTER(CConfig)]),
    "vvli_gpu_storage_element_count": (c_uint64, [POINTER(CConfig)]),
    "vvli_gpu_model_create": (c_int, [POINTER(CConfig), c_uint32, c_void_p, c_size_t, POINTER(c_void_p)]),
    "vvli_gpu_model_destroy": (c_int, [c_void_p]),
    "vvli_gpu_moe_storage_element_count": (c_uint64, [POINTER(CConfig)]),
    "vvli_gpu_model_create_from_safetensors": (
        c_int, [POINTER(CConfig), c_uint32, c_void_p, c_size_t, PROGRESS_FN, c_void_p, POINTER(c_void_p)]),
    "vvli_gpu_model_create_from_gguf": (
        c_int, [c_void_p, c_size_t, c_uint32, c_uint32, PROGRESS_FN, c_void_p, POINTER(CConfig), POINTER(c_void_p)]),
    "vvli_gpu_read_weights": (c_int, [c_void_p, c_uint64, c_uint64, c_void_p]),
    "vvli_gpu_moe_model_create": (c_int, [POINTER(CConfig), c_uint32, c_void_p, c_size_t, POINTER(c_void_p)]),
    "vvli_gpu_kv_clear": (c_int, [c_void_p]),
    "vvli_gpu_set_rope_table": (c_int, [c_void_p, c_void_p, c_uint32]),
    "vvli_gpu_forward_token": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, POINTER(c_uint32)]),
    "vvli_gpu_forward_token_view": (c_int, [c_void_p, c_uint32, c_uint32, POINTER(c_void_p), POINTER(c_uint32)]),
    "vvli_gpu_set_resident": (c_int, [c_void_p, c_uint32]),
    "vvli_gpu_forward_embedding": (c_int, [c_void_p, c_void_p, c_uint32, c_void_p, POINTER(c_uint32)]),
    "vvli_gpu_forward_token_debug": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
    "vvli_gpu_kv_read": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
    "vvli_gpu_prefill": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_void_p, POINTER(c_uint32)]),
    "vvli_gpu_generate_greedy": (
        c_int,
        [c_void_p, c_void_p, c_uint32, c_uint32, c_int64, c_uint32, c_void_p, POINTER(c_uint32), POINTER(CStats)],
    ),
    "vvli_gpu_generate": (
        c_int,
        [c_void_p, c_void_p, c_uint32, c_uint32, c_int64, c_uint32, POINTER(CSampling), c_void_p, POINTER(c_uint32),
         POINTER(CStats)],
    ),
    "vvli_gpu_sampler_next": (
        c_int, [c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, POINTER(CSampling), c_void_p,
                POINTER(c_uint32)]),
    "vvli_gpu_prng_seed": (None, [c_uint64, c_void_p]),
    "vvli_gpu_profile_step": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_uint32, POINTER(c_uint32)]),
    "vvli_gpu_set_decode_path": (c_int, [c_void_p, c_uint32]),
    "vvli_gpu_set_prefill_path": (c_int, [c_void_p, c_uint32]),
    "vvli_gpu_profile_persistent": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_uint32, POINTER(c_uint32)]),
    "vvli_gpu_last_launch_time": (c_int, [c_void_p, POINTER(ctypes.c_float)]),
    "vvli_gpu_test_inject_step_error": (c_int, [c_void_p, c_uint32]),
    "vvli_gpu_test_set_prefill_attention_form": (c_int, [ctypes.c_int32]),
    "vvli_gpu_test_sampler_trace": (
        c_int, [c_void_p, c_uint32, POINTER(CSampling), c_void_p, POINTER(c_uint32), c_void_p, c_void_p, c_void_p,
                POINTER(c_uint32)]),
    "vvli_gpu_linear": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_void_p]),
    "vvli_gpu_linear_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                                        c_void_p]),
    "vvli_host_fill_deterministic": (None, [c_void_p, c_size_t, c_uint32]),
    "vvli_host_fill_synthetic": (c_int, [POINTER(CConfig), c_uint64, c_float, c_void_p, c_size_t, c_uint32]),
    "vvli_host_synthetic_normal": (c_double, [c_uint64, c_uint64, c_uint64]),
    "vvli_host_llama3_inv_freq": (c_int, [c_uint32, c_float, c_float, c_float, c_float, c_uint32, c_void_p]),
    "vvli_host_config_from_json": (c_int, [c_char_p, c_size_t, c_uint32, POINTER(CConfig)]),
    "vvli_host_config_from_gguf": (c_int, [c_void_p, c_size_t, c_uint32, POINTER(CConfig)]),
    "vvli_host_load_safetensors": (
        c_int, [POINTER(CConfig), c_void_p, c_size_t, c_void_p, c_size_t, PROGRESS_FN, c_void_p]),
    "vvli_host_load_gguf": (c_int, [POINTER(CConfig), c_void_p, c_size_t, c_void_p, c_size_t, PROGRESS_FN, c_void_p]),
    "vvli_host_map_file": (c_int, [c_char_p, POINTER(c_void_p), POINTER(c_size_t)]),
    "vvli_host_unmap_file": (c_int, [c_void_p, c_size_t]),
    "vvli_host_f16_to_f32": (c_float, [ctypes.c_uint16]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libvvli_gpu.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with make -C vvli_amd/csrc")
        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | getattr(os, "RTLD_GLOBAL", 0))
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.vvli_gpu_abi_version() != ABI_VERSION:
            raise RuntimeError("libvvli_gpu.so ABI version mismatch")
        _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().vvli_gpu_last_error() or b""
        raise VvliError(rc, msg.decode(errors="replace"))
