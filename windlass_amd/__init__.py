"""windlass_amd — the MoE-layer hot path of windlass (GLM-5.2 decode), native
to MI355X (gfx950): hand-written HIP kernels behind the C ABI declared in
include/windlass_moe.h, with a thin ctypes binding in windlass_amd.moe."""
__all__ = ["moe", "hip"]
