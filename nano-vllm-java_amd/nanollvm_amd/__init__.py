"""MI355X (gfx950) paged attention for nano-vllm-java: host mirror of the reference's attention
boundary over the C-ABI library libnva.so.  ``step`` binds the library's step-metadata
producers; ``workloads`` builds the synthetic workloads of the benchmark and tests."""

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
