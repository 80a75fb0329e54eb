"""MI355X-native ResidualQuant packed KV-cache path.

Hand-written gfx950 HIP kernels behind a C ABI (``include/rq_hip.h``,
``librq_hip.so``), with the reference plugin's operator surface on top:
``quantize(...)`` and ``attention(...)`` take the same arguments as
``residual_quantization._cuda.{quantize, attention}``
(plugins/residual_quantization/csrc/dispatch/binding.cpp:19-38).
"""

from .ops import attention, dequantize, paged_attention_bf16, quantize  # noqa: F401
from .layout import page_width  # noqa: F401
from .group import DeferredKVGroup  # noqa: F401

__all__ = ("attention", "quantize", "dequantize", "paged_attention_bf16", "page_width",
           "DeferredKVGroup")
