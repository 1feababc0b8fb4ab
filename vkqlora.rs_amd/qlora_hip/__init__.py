"""qlora_hip -- MI355X (gfx950) QloraLinear hot path behind a C ABI.

Python mirror of stuarch/VkQLoRA.rs's ``qlora_wgpu`` module
(qlora-python/src/lib.rs) plus numpy-level helpers; every call runs the
hand-written HIP kernels of ``libqlora_hip.so``.
"""
from ._lib import (Context, NoDevice, QloraError, default_context, load,  # noqa
                   LIB_PATH, EXPORTED)
from .api import (Adam8bit, BackwardOut, PagedAdam, QuantizedWeight,  # noqa
                  backward, block_scales, dequantize, forward, matmul,
                  matmul_trans_a, matmul_trans_b, qlora_linear_backward,
                  qlora_linear_forward, quantize, quantize_nf4, qweight_struct,
                  storage_bytes, nf4_file_bytes, save_nf4, load_nf4, nf4_file_views)

__all__ = [
    "quantize_nf4", "qlora_linear_forward", "qlora_linear_backward",
    "QuantizedWeight", "BackwardOut", "PagedAdam", "Adam8bit", "Context",
    "QloraError", "NoDevice", "quantize", "dequantize", "block_scales",
    "forward", "backward", "matmul", "matmul_trans_a", "matmul_trans_b",
    "storage_bytes", "nf4_file_bytes", "save_nf4", "load_nf4", "nf4_file_views",
]
