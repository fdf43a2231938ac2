"""MI355X-native hot-path operators of the Qwen3 layer (RPGBarEngine operator layer).

The product is librpg_ops.so (HIP, gfx950) with the C ABI of include/rpg_ops.h;
`ops` is the host-side mirror of the reference operator layer over it.
"""
from . import ops  # noqa: F401
from .ops import RpgError  # noqa: F401

__all__ = ["ops", "RpgError"]
