"""openattention_amd -- OpenAttention's sparse decode path on MI355X (gfx950).

Host side in Python on PyTorch-ROCm; the compute is hand-written HIP kernels behind a C ABI
(include/openattention_amd.h), loaded by ctypes (openattention_amd.lib).

    from openattention_amd import ours_flash, decode_expand_attention, OursHIP
"""
from openattention_amd.ops import decode_expand_attention, ours_flash  # noqa: F401
from openattention_amd.method import C, Ctx, OursHIP, attn_hook  # noqa: F401

__all__ = ["ours_flash", "decode_expand_attention", "OursHIP", "Ctx", "C", "attn_hook"]
