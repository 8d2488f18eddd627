"""MI355X (gfx950) paged attention for nano-vllm-java: host mirror of the reference's attention
boundary over the C-ABI library libnva.so.  ``engine`` holds the host-side metadata producers
(block tables, slot mappings, cu_seqlens) and the synthetic workloads."""

from . import _native  # noqa: F401
from .layers import (  # noqa: F401
    Attention,
    Context,
    IllegalArgumentException,
    IllegalStateException,
    KvCacheArena,
    Linear,
    NullPointerException,
    NvaError,
    RMSNorm,
    RotaryEmbedding,
    UnsupportedShapeError,
)
