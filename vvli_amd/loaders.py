"""Checkpoint loaders: HF ``config.json`` + ``model.safetensors`` directories and
GGUF files into the contiguous weight blob ``Runner`` takes.

Mirrors ``llm.loadOwnedFromDirectory`` / ``loadOwnedFromSafetensorsFile`` /
``loadOwnedFromGgufFile`` (src/llm.zig:839-921). Parsing, name lookup and dtype
conversion run in libvvli_gpu.so (``vvli_host_load_*``); files are memory-mapped
read-only, as the reference maps them.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import byref, c_size_t, c_void_p
from typing import Callable, Optional

import numpy as np

from . import _lib
from .config import WEIGHT_BF16, Config
from .runtime import empty_blob

Progress = Optional[Callable[[int, int, str], None]]


class MappedFile:
    """A whole file mapped read-only (vvli_host_map_file); use as a context manager."""

    def __init__(self, path: str | os.PathLike):
        self.ptr = c_void_p()
        self.size = c_size_t()
        _lib.check(_lib.lib().vvli_host_map_file(os.fsencode(path), byref(self.ptr), byref(self.size)))

    def close(self) -> None:
        if self.ptr:
            _lib.check(_lib.lib().vvli_host_unmap_file(self.ptr, self.size))
            self.ptr = c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _callback(progress: Progress):
    if progress is None:
        return ctypes.cast(None, _lib.PROGRESS_FN)
    return _lib.PROGRESS_FN(lambda _u, done, total, name: progress(done, total, name.decode()))


def _image(data) -> tuple[c_void_p, int, np.ndarray]:
    buf = np.frombuffer(data, dtype=np.uint8)
    return c_void_p(buf.ctypes.data), buf.size, buf


def safetensors_into_blob(cfg: Config, data, weight_kind: int = WEIGHT_BF16, progress: Progress = None) -> np.ndarray:
    """loadSafetensorsIntoOwnedModel (src/llm.zig:923-1006) over an in-memory image."""
    ptr, n, _keep = _image(data)
    return _load_safetensors(cfg, ptr, n, weight_kind, progress)


def gguf_into_blob(data, weight_kind: int = WEIGHT_BF16, progress: Progress = None) -> tuple[Config, np.ndarray]:
    """Config.fromGguf + loadGgufIntoOwnedModel (src/llm.zig:153-193, 1008-1065)
    over an in-memory GGUF image."""
    ptr, n, _keep = _image(data)
    return _load_gguf(ptr, n, weight_kind, progress)


def load_safetensors(cfg: Config, path: str | os.PathLike, weight_kind: int = WEIGHT_BF16,
                     progress: Progress = None) -> np.ndarray:
    """loadOwnedFromSafetensorsFile (src/llm.zig:849-883)."""
    with MappedFile(path) as f:
        return _load_safetensors(cfg, f.ptr, f.size.value, weight_kind, progress)


def load_directory(model_dir: str | os.PathLike, weight_kind: int = WEIGHT_BF16,
                   progress: Progress = None) -> tuple[Config, np.ndarray]:
    """loadOwnedFromDirectory (src/llm.zig:839-847): config.json + model.safetensors."""
    with open(os.path.join(model_dir, "config.json"), "rb") as fh:
        cfg = Config.from_json(fh.read())
    return cfg, load_safetensors(cfg, os.path.join(model_dir, "model.safetensors"), weight_kind, progress)


def load_gguf(path: str | os.PathLike, weight_kind: int = WEIGHT_BF16,
              progress: Progress = None) -> tuple[Config, np.ndarray]:
    """loadOwnedFromGgufFile (src/llm.zig:885-921)."""
    with MappedFile(path) as f:
        return _load_gguf(f.ptr, f.size.value, weight_kind, progress)


def device_load_safetensors(cfg: Config, path: str | os.PathLike, max_seq_len: int, weight_kind: int = WEIGHT_BF16,
                            progress: Progress = None):
    """A Runner whose weights went from the mapped file straight to HBM
    (vvli_gpu_model_create_from_safetensors): no host blob."""
    from .runtime import Runner

    with MappedFile(path) as f:
        c = cfg.to_c(weight_kind)
        h = c_void_p()
        _lib.check(_lib.lib().vvli_gpu_model_create_from_safetensors(byref(c), max_seq_len, f.ptr, f.size.value,
                                                                     _callback(progress), None, byref(h)))
    return Runner.from_handle(cfg, h, max_seq_len, weight_kind)


def device_load_directory(model_dir: str | os.PathLike, max_seq_len: int, weight_kind: int = WEIGHT_BF16,
                          progress: Progress = None):
    """config.json + model.safetensors straight to HBM; returns (Config, Runner)."""
    with open(os.path.join(model_dir, "config.json"), "rb") as fh:
        cfg = Config.from_json(fh.read())
    return cfg, device_load_safetensors(cfg, os.path.join(model_dir, "model.safetensors"), max_seq_len, weight_kind,
                                        progress)


def device_load_gguf(path: str | os.PathLike, max_seq_len: int, weight_kind: int = WEIGHT_BF16,
                     progress: Progress = None):
    """A GGUF file straight to HBM (vvli_gpu_model_create_from_gguf); returns (Config, Runner)."""
    from .runtime import Runner

    with MappedFile(path) as f:
        c = _lib.CConfig()
        h = c_void_p()
        _lib.check(_lib.lib().vvli_gpu_model_create_from_gguf(f.ptr, f.size.value, weight_kind, max_seq_len,
                                                              _callback(progress), None, byref(c), byref(h)))
    cfg = Config.from_c(c)
    return cfg, Runner.from_handle(cfg, h, max_seq_len, weight_kind)


def _load_safetensors(cfg, ptr, n, weight_kind, progress):
    blob = empty_blob(cfg, weight_kind)
    c = cfg.to_c(weight_kind)
    cb = _callback(progress)
    _lib.check(_lib.lib().vvli_host_load_safetensors(byref(c), ptr, n, c_void_p(blob.ctypes.data), blob.size, cb,
                                                     None))
    return blob


def _load_gguf(ptr, n, weight_kind, progress):
    c = _lib.CConfig()
    _lib.check(_lib.lib().vvli_host_config_from_gguf(ptr, n, weight_kind, byref(c)))
    cfg = Config.from_c(c)
    blob = empty_blob(cfg, weight_kind)
    cb = _callback(progress)
    _lib.check(_lib.lib().vvli_host_load_gguf(byref(c), ptr, n, c_void_p(blob.ctypes.data), blob.size, cb, None))
    return cfg, blob
