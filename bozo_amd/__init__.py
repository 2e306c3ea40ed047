"""bozo_amd -- MI355X-native (gfx950) sigmoid-tension op of TensionLM.

Hand-written HIP kernels behind a C ABI (include/tension_hip.h,
bozo_amd/lib/libtension_hip.so), bound with ctypes under torch autograd.
``causal_tension`` is the drop-in for the reference's
``triton_tension.causal_tension``.
"""
from .ops import (TensionDecodeCache, causal_tension, decode_step, global_tension,  # noqa: F401
                  rope)

__all__ = ["causal_tension", "global_tension", "decode_step", "TensionDecodeCache", "rope"]
