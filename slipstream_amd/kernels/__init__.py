"""HIP (gfx950) kernels behind the reference's ``slipstream.kernels`` call signatures."""

from slipstream_amd.kernels.block_copy import copy_blocks, swap_blocks
from slipstream_amd.kernels.paged_attention import (
    attention_status,
    paged_attention,
    paged_attention_decode,
    paged_attention_prefill,
    paged_attention_shared_prefix,
    paged_attention_varlen,
)
from slipstream_amd.kernels.norm_act import fused_rmsnorm, fused_swiglu
from slipstream_amd.kernels.packed_step import packed_attention
from slipstream_amd.kernels.quant_gemm import w4a16_gemm
from slipstream_amd.kernels.reshape_and_cache import reshape_and_cache
from slipstream_amd.kernels.rope_cache import rope_and_cache

__all__ = [
    "attention_status",
    "copy_blocks",
    "fused_rmsnorm",
    "fused_swiglu",
    "packed_attention",
    "paged_attention",
    "paged_attention_decode",
    "paged_attention_prefill",
    "paged_attention_shared_prefix",
    "paged_attention_varlen",
    "reshape_and_cache",
    "rope_and_cache",
    "swap_blocks",
    "w4a16_gemm",
]
