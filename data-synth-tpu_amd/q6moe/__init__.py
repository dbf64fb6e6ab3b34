"""q6moe: MI355X-native packed-weight expert matmul and INT8 KV cache.

GGUF expert tables (Q6_K, Q5_K, Q4_K, Q8_0 gate/up; those or Q5_1 down) are
decoded inside the matmul kernels. Host surface mirrors the reference
operators of AhmadSaeedZaidi/data-synth-tpu:

* ``pack_q6`` / ``unpack_q6`` / ``PackedQ6``   (kaggle/packed_q6/layout.py)
* ``q6_matmul``                                (kaggle/packed_q6/kernel.py)
* ``block_layout`` / ``dequantize_rows``       (kaggle/glm53_offload/gguf_quant.py)
* ``expert_parallel`` / ``grouped_expert_parallel`` (kaggle/qwen38_tpu/experts.py,
  grouped_experts.py); ``routes`` (math.py:277-281)
* ``q8_matmul`` / ``bf16_q8_matmul`` / ``pack_q8`` (kaggle/qwen38_tpu/compute.py)
* ``quantize`` / ``write_quantized`` / ``gather_scale_plane`` /
  ``read_quantized`` (kaggle/qwen38_tpu/attention_cache.py), with the paged
  forms ``write_paged`` / ``read_paged`` and ``paged_decode_attention``

All device work runs in hand-written HIP kernels (libq6moe.so, gfx950).
"""

from .layout import LAYOUT, PackedQ6, pack_q6, pack_q6_experts, unpack_q6

__all__ = ["LAYOUT", "PackedQ6", "pack_q6", "pack_q6_experts", "unpack_q6"]


def __getattr__(name):
    # Torch-dependent operators load lazily so the packers stay importable
    # (and fast) without initialising torch.
    if name in ("q6_matmul", "q6_decode", "q6_pack"):
        from . import kernel

        return getattr(kernel, name)
    if name in ("block_layout", "dequantize_rows"):
        from . import quant

        return getattr(quant, name)
    if name in ("expert_parallel", "grouped_expert_parallel", "pack_experts"):
        from . import experts

        return getattr(experts, name)
    if name in ("q8_matmul", "bf16_q8_matmul", "pack_q8"):
        from . import compute

        return getattr(compute, name)
    if name in ("quantize", "write_quantized", "gather_scale_plane", "read_quantized", "write_paged", "read_paged",
                "paged_decode_attention"):
        from . import attention_cache

        return getattr(attention_cache, name)
    if name == "routes":
        from . import router

        return router.routes
    raise AttributeError(name)
