"""vvli_amd: MI355X (gfx950) dense-decoder forward pass for VVLI.

The product is libvvli_gpu.so (C ABI in include/vvli_gpu.h and
include/vvli_host.h); this package is a thin Python host over it.
"""
from ._lib import LIB_PATH, VvliError  # noqa: F401
from .config import Config, NAMED, WEIGHT_BF16, WEIGHT_F32  # noqa: F401
