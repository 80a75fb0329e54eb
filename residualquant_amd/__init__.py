"""MI355X-native ResidualQuant packed KV-cache path.

Hand-written gfx950 HIP kernels behind a C ABI (``include/rq_hip.h``,
``librq_hip.so``), with the reference plugin's operator surface on top:
``quantize(...)`` and ``attention(...)`` take the same arguments as
``residual_quantization._cuda.{quantize, attention}``
(plugins/residual_quantization/csrc/dispatch/binding.cpp:19-38), and
``flash_attn_varlen_func(...)`` takes the keywords of the full-prompt call in
src/residual_quantization/packed_backend.py:63-77.
"""

from .ops import (attention, dequantize, flash_attn_varlen_func, packed_prefill_attention,  # noqa: F401
                  paged_attention_bf16, prefill_attention, quantize)
from .layout import page_width  # noqa: F401
from .group import DeferredKVGroup  # noqa: F401

__all__ = ("attention", "quantize", "dequantize", "flash_attn_varlen_func", "prefill_attention",
           "packed_prefill_attention",
           "paged_attention_bf16", "page_width", "DeferredKVGroup")
