"""The C-ABI library loads without a GPU and exports every entry point the
headers in include/ declare; the ctypes binding covers all of them."""
import ctypes
import re
from pathlib import Path

from vvli_amd import _lib

INCLUDE = Path(__file__).resolve().parents[1] / "include"
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(vvli_\w+)\s*\(", re.M)


def declared_functions() -> set:
    names = set()
    for h in INCLUDE.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(DECL.findall(text))
    return names


def test_headers_declare_entry_points():
    names = declared_functions()
    assert "vvli_gpu_model_create" in names and "vvli_gpu_forward_token" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert declared_functions() <= set(_lib.PROTOTYPES)


def test_abi_version_and_error_text():
    lib = _lib.lib()
    assert lib.vvli_gpu_abi_version() == _lib.ABI_VERSION
    # A NULL config is rejected on the host, with a message.
    assert lib.vvli_gpu_config_validate(None) == 100
    assert b"NULL" in lib.vvli_gpu_last_error()


def test_create_rejects_bad_input_without_a_gpu():
    from vvli_amd import config as C

    cfg = C.tiny_test()
    c = cfg.to_c(C.WEIGHT_F32)
    h = ctypes.c_void_p()
    lib = _lib.lib()
    # max_seq_len beyond max_position_embeddings: KVCache.init's InvalidConfig (src/llm.zig:548).
    assert lib.vvli_gpu_model_create(ctypes.byref(c), 17, ctypes.c_void_p(1), 10**6, ctypes.byref(h)) == 1
    assert lib.vvli_gpu_model_create(ctypes.byref(c), 8, None, 10, ctypes.byref(h)) == 100
