"""HIP (gfx950) kernels behind the reference's ``slipstream.kernels`` call signatures."""

from slipstream_amd.kernels.paged_attention import (
    paged_attention,
    paged_attention_decode,
    paged_attention_prefill,
    paged_attention_varlen,
)
from slipstream_amd.kernels.quant_gemm import w4a16_gemm
from slipstream_amd.kernels.reshape_and_cache import reshape_and_cache

__all__ = [
    "paged_attention",
    "paged_attention_decode",
    "paged_attention_prefill",
    "paged_attention_varlen",
    "reshape_and_cache",
    "w4a16_gemm",
]
