"""MI355X-native (gfx950) implementation of emberlm's activation-memory hot path.

Native pieces (built in-tree by ``python -m emberlm_amd.build``):
  lib/libember_hip.so  gfx950 kernels behind the C ABI of include/ember_hip.h
  lib/libctd.so        C++ Tensor / autograd / Module / AdamW layer (include/ctd/)
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
