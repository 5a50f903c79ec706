"""slipstream_amd: MI355X (gfx950) ragged paged-attention path for slipstream.

The package replaces the reference's hot path (``slipstream/kernels``): the
KV-cache scatter, paged-attention decode and chunked prefill, a packed
(varlen) mixed step and the W4A16 int4 linear, each a hand-written HIP kernel
called through the C ABI in ``include/slipstream_hip.h``.
"""

__version__ = "0.1.0"
