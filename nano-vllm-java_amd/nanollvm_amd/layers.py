"""Host-side mirror of nano-vllm-java's attention boundary over libnva.so.

Class and method names follow the reference so that callers (and the parity tests) read like
the reference's own code:

* ``Context``        -- internal/Context.java (step metadata; ``set``/``clear``) plus the device
                        and stream the native context owns.
* ``KvCacheArena``   -- engine/KvCacheArena.java (per-layer K/V pages, resident in HBM).
* ``RotaryEmbedding``-- layers/Norms.java:158-388 (cos|sin table, ``forward``).
* ``Attention``      -- layers/Attention.java (constructor arguments, ``forward``).
* ``RMSNorm``        -- layers/Norms.java:32-97 (``forward``; ``weightless``), applied per head
                        by the model layers before RoPE.
* ``Linear``         -- layers/Linear.java Linear.Row (``forward``): o_proj on the attention
                        output.

(Reference paths are relative to nano-vllm-java/src/main/java/com/igormaznitsa/nanollvm/.)
Tensors are torch CUDA float32 tensors (device memory only; torch does no compute here).  Java
exceptions map to Python exceptions of the same names.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native as N


class NvaError(RuntimeError):
    """Any failure reported by libnva.so."""


class IllegalArgumentException(NvaError, ValueError):
    pass


class IllegalStateException(NvaError):
    pass


class NullPointerException(NvaError, TypeError):
    pass


class UnsupportedShapeError(NvaError, NotImplementedError):
    pass


_EXC = {
    N.NVA_E_ARG: IllegalArgumentException,
    N.NVA_E_LAYER: IllegalArgumentException,
    N.NVA_E_ROPE_POS: IllegalArgumentException,
    N.NVA_E_SHARED_KV: IllegalStateException,
    N.NVA_E_NO_ARENA: NullPointerException,
    N.NVA_E_NO_STEP: NullPointerException,
    N.NVA_E_UNSUPPORTED: UnsupportedShapeError,
}


def _check(ctx_handle, status: int, what: str) -> None:
    if status == N.NVA_OK:
        return
    lib = N.load()
    msg = lib.nva_last_error(ctx_handle) if ctx_handle else None
    msg = msg.decode() if msg else lib.nva_status_string(status).decode()
    raise _EXC.get(status, NvaError)(f"{what}: {msg}")


def _i32(a) -> Optional[np.ndarray]:
    if a is None:
        return None
    return np.ascontiguousarray(np.asarray(a), dtype=np.int32)


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _dev(t: Optional[torch.Tensor], name: str):
    if t is None:
        return None
    if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
        raise IllegalArgumentException(f"{name} must be a contiguous float32 device tensor")
    return t.data_ptr()


class Context:
    """Context.java plus the native context (device, stream, step buffers).

    ``stream`` defaults to torch's current stream on the device so that the library's kernels
    are ordered with the caller's torch work."""

    def __init__(self, device: int = 0, stream: Optional[torch.cuda.Stream] = None):
        lib = N.load()
        h = ctypes.c_void_p()
        st = lib.nva_ctx_create(device, ctypes.byref(h))
        if st != N.NVA_OK:
            raise NvaError(f"nva_ctx_create(device={device}) failed: "
                           f"{lib.nva_status_string(st).decode()} (no usable HIP device?)")
        self._h = h
        self.device = device
        self._kv = None
        self._positions_key = None
        s = stream if stream is not None else torch.cuda.current_stream(device)
        _check(self._h, lib.nva_ctx_set_stream(self._h, ctypes.c_void_p(s.cuda_stream)),
               "set_stream")
        self._stream = s

    @property
    def handle(self):
        return self._h

    def set_stream(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Run the context's work on ``stream`` (default: torch's current stream), e.g. the
        stream a HIP graph is being captured on."""
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        _check(self._h, N.load().nva_ctx_set_stream(self._h, ctypes.c_void_p(s.cuda_stream)),
               "set_stream")
        self._stream = s

    # ---- Context.java API
    def bind_kv_cache(self, arena: "KvCacheArena") -> None:
        self._kv = arena

    def kv_cache(self) -> Optional["KvCacheArena"]:
        return self._kv

    def set(self, is_prefill: bool, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q: int = 0,
            max_seqlen_k: int = 0, slot_mapping=None, context_lens=None, block_tables=None,
            seq_ids=None, positions=None) -> None:
        """Context.set (Context.java:39-59); ``block_tables`` is a list of per-sequence lists or
        a 2-D array, padded with -1 (Transformer.prepareBlockTables); ``positions`` is the
        step's float positions tensor."""
        cu_q, cu_k = _i32(cu_seqlens_q), _i32(cu_seqlens_k)
        slots = _i32(slot_mapping)
        lens = _i32(context_lens)
        bt = None
        stride = 0
        if block_tables is not None:
            if isinstance(block_tables, np.ndarray):
                bt = np.ascontiguousarray(block_tables, dtype=np.int32)
            else:
                width = max((len(r) for r in block_tables), default=0)
                bt = np.full((len(block_tables), max(width, 1)), -1, np.int32)
                for i, r in enumerate(block_tables):
                    bt[i, :len(r)] = r
            if bt.ndim != 2:
                raise IllegalArgumentException("block tables must be 2-D")
            if bt.shape[1] == 0:
                bt = np.full((bt.shape[0], 1), -1, np.int32)
            stride = bt.shape[1]
        if is_prefill:
            num_seqs = 0 if cu_q is None else len(cu_q) - 1
        else:
            num_seqs = 0 if lens is None else len(lens)
        ids = _i32(seq_ids)
        pos = None if positions is None else np.ascontiguousarray(
            positions.detach().cpu().numpy() if isinstance(positions, torch.Tensor) else positions,
            dtype=np.float32)
        ntok = len(pos) if pos is not None else (len(ids) if ids is not None else 0)
        lib = N.load()
        _check(self._h, lib.nva_step_set(
            self._h, int(bool(is_prefill)), _ptr(cu_q), _ptr(cu_k), num_seqs, int(max_seqlen_q),
            int(max_seqlen_k), _ptr(slots), 0 if slots is None else len(slots), _ptr(lens),
            _ptr(bt), stride, _ptr(ids), _ptr(pos), ntok), "Context.set")
        self._positions_key = None if pos is None else pos.tobytes()

    def prepare_prefill(self, seqs, block_size: int) -> None:
        """Transformer.preparePrefill + Context.set (Transformer.java:342-418) in the library:
        ``seqs`` are Sequence-like objects (engine/Sequence.java) with numCachedTokens /
        numScheduledTokens set."""
        from .step import seq_array
        arr, keep = seq_array(seqs)
        _check(self._h, N.load().nva_step_prepare_prefill(self._h, arr, len(seqs), block_size),
               "Transformer.preparePrefill")
        del keep
        self._positions_key = None

    def prepare_decode(self, seqs, block_size: int) -> None:
        """Transformer.prepareDecode + Context.set (Transformer.java:427-456) in the library."""
        from .step import seq_array
        arr, keep = seq_array(seqs)
        _check(self._h, N.load().nva_step_prepare_decode(self._h, arr, len(seqs), block_size),
               "Transformer.prepareDecode")
        del keep
        self._positions_key = None

    def set_positions(self, positions) -> None:
        pos = np.ascontiguousarray(
            positions.detach().cpu().numpy() if isinstance(positions, torch.Tensor) else positions,
            dtype=np.float32)
        key = pos.tobytes()
        if key == self._positions_key:
            return
        lib = N.load()
        _check(self._h, lib.nva_step_positions(self._h, _ptr(pos), len(pos)), "positions")
        self._positions_key = key

    def clear(self) -> None:
        N.load().nva_step_clear(self._h)
        self._kv = None
        self._positions_key = None

    # ---- native extras
    def sync(self) -> None:
        _check(self._h, N.load().nva_ctx_sync(self._h), "sync")

    def set_timing(self, enable: bool) -> None:
        _check(self._h, N.load().nva_ctx_set_timing(self._h, int(bool(enable))), "timing")

    def kernel_stats(self, kernel: str):
        n = ctypes.c_int64()
        ms = ctypes.c_double()
        _check(self._h, N.load().nva_ctx_kernel_stats(self._h, kernel.encode(), ctypes.byref(n),
                                                        ctypes.byref(ms)), "kernel_stats")
        return n.value, ms.value

    def reset_stats(self) -> None:
        _check(self._h, N.load().nva_ctx_reset_stats(self._h), "reset_stats")

    def close(self) -> None:
        if self._h:
            N.load().nva_ctx_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class KvCacheArena:
    """KvCacheArena(numLayers, numBlocks, blockSize, numKvHeads, headDim) or, with per-layer
    ``head_dims``/``allocate``, KvCacheArena(numBlocks, blockSize, numKvHeads, headDims[],
    allocateLayer[]) (KvCacheArena.java:41-90).  Pages live in HBM, zero-filled."""

    def __init__(self, ctx: Context, num_layers: int, num_blocks: int, block_size: int,
                 num_kv_heads: int, head_dim: int = 0, head_dims: Sequence[int] = None,
                 allocate: Sequence[bool] = None):
        if head_dims is None:
            head_dims = [head_dim] * num_layers
        if allocate is None:
            allocate = [True] * len(head_dims)
        if len(head_dims) != len(allocate):
            raise IllegalArgumentException("headDims and allocateLayer length mismatch")
        hd = np.asarray(head_dims, np.int32)
        al = np.asarray([1 if a else 0 for a in allocate], np.uint8)
        h = ctypes.c_void_p()
        lib = N.load()
        _check(ctx.handle, lib.nva_kv_create(ctx.handle, len(hd), num_blocks, block_size,
                                             num_kv_heads, _ptr(hd), _ptr(al), ctypes.byref(h)),
               "KvCacheArena")
        self._h = h
        self._ctx = ctx
        self.num_layers = len(hd)
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dims = list(head_dims)

    @property
    def handle(self):
        return self._h

    @staticmethod
    def blocks_that_fit(ctx: Context, num_layers: int, block_size: int, num_kv_heads: int,
                        head_dim: int = 0, head_dims: Sequence[int] = None,
                        allocate: Sequence[bool] = None, fraction: float = 0.9):
        """(pages that fit in ``fraction`` of the device's free HBM, the free bytes it used):
        the heap cap of Config.resolveNumKvcacheBlocks (Config.java:93-125) with HBM in place of
        the Java heap."""
        if head_dims is None:
            head_dims = [head_dim] * num_layers
        if allocate is None:
            allocate = [True] * len(head_dims)
        hd = np.asarray(head_dims, np.int32)
        al = np.asarray([1 if a else 0 for a in allocate], np.uint8)
        blocks = ctypes.c_int()
        free = ctypes.c_int64()
        _check(ctx.handle, N.load().nva_kv_blocks_that_fit(
            ctx.handle, len(hd), block_size, num_kv_heads, _ptr(hd), _ptr(al),
            ctypes.c_float(fraction), ctypes.byref(blocks), ctypes.byref(free)),
            "KvCacheArena.blocks_that_fit")
        return blocks.value, free.value

    @staticmethod
    def resolve_num_blocks(ctx: Context, configured: int, max_num_seqs: int, max_model_len: int,
                           block_size: int, num_kv_heads: int, head_dims: Sequence[int],
                           allocate: Sequence[bool] = None, fraction: float = 0.9) -> int:
        """Config.resolveNumKvcacheBlocks (Config.java:93-125) for a device arena: the configured
        count if positive, else min(max(maxNumSeqs * ceil(maxModelLen / blockSize), 128), the
        pages that fit in ``fraction`` of the free HBM)."""
        if configured > 0:
            return configured
        per_seq = (max_model_len + block_size - 1) // block_size
        estimated = max(max_num_seqs * per_seq, 128)
        cap, _ = KvCacheArena.blocks_that_fit(ctx, len(head_dims), block_size, num_kv_heads,
                                              head_dims=head_dims, allocate=allocate,
                                              fraction=fraction)
        return min(estimated, cap)

    def _layer(self, layer: int):
        k = ctypes.c_void_p()
        v = ctypes.c_void_p()
        n = ctypes.c_int64()
        _check(self._ctx.handle, N.load().nva_kv_layer(self._h, layer, ctypes.byref(k),
                                                       ctypes.byref(v), ctypes.byref(n)),
               "KvCacheArena layer")
        return k.value, v.value, n.value

    def shape(self, layer: int):
        return (self.num_blocks, self.block_size, self.num_kv_heads, self.head_dims[layer])

    def get_key_cache(self, layer: int) -> np.ndarray:
        """Host copy of layer's K pages ([numBlocks, blockSize, Hkv, d])."""
        return self.read(layer, 0)

    def get_value_cache(self, layer: int) -> np.ndarray:
        return self.read(layer, 1)

    def read(self, layer: int, which: int, offset: int = 0, count: int = None) -> np.ndarray:
        _, _, nbytes = self._layer(layer)
        total = nbytes // 4
        count = total - offset if count is None else count
        out = np.empty(count, np.float32)
        _check(self._ctx.handle, N.load().nva_kv_read(self._h, layer, which, offset, _ptr(out),
                                                      count), "KvCacheArena read")
        if offset == 0 and count == total:
            return out.reshape(self.shape(layer))
        return out

    def write(self, layer: int, which: int, data: np.ndarray, offset: int = 0) -> None:
        data = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        _check(self._ctx.handle, N.load().nva_kv_write(self._h, layer, which, offset,
                                                       _ptr(data), data.size),
               "KvCacheArena write")

    def device_ptrs(self, layer: int):
        k, v, n = self._layer(layer)
        return k, v, n

    def close(self) -> None:
        if self._h:
            N.load().nva_kv_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class RotaryEmbedding:
    """RotaryEmbedding(headSize, rotaryDim, maxPositionEmbeddings, base) (Norms.java:171-205).

    ``cos_sin`` may pass the caller's own [maxPos, headSize] table (the Java table); otherwise
    the library builds it with the reference's arithmetic."""

    def __init__(self, ctx: Context, head_size: int, rotary_dim: int, max_position_embeddings: int,
                 base: float, cos_sin: Optional[np.ndarray] = None):
        lib = N.load()
        h = ctypes.c_void_p()
        if cos_sin is not None:
            t = np.ascontiguousarray(cos_sin, dtype=np.float32)
            if t.shape != (max_position_embeddings, head_size):
                raise IllegalArgumentException("cos_sin must be [maxPos, headSize]")
            st = lib.nva_rope_create(ctx.handle, _ptr(t), max_position_embeddings, head_size,
                                     ctypes.byref(h))
        else:
            st = lib.nva_rope_create_theta(ctx.handle, head_size, rotary_dim,
                                           max_position_embeddings,
                                           float(np.float32(base)), ctypes.byref(h))
        _check(ctx.handle, st, "RotaryEmbedding")
        self._h = h
        self.head_size = head_size
        self.max_position = max_position_embeddings

    @property
    def handle(self):
        return self._h

    def forward(self, positions, query: torch.Tensor, key: torch.Tensor, ctx: Context):
        """RotaryEmbedding.forward(positions, query, key, context) -> (q_rot, k_rot)."""
        if positions is not None:
            ctx.set_positions(positions)
        if query.dim() != 3 or key.dim() != 3:
            raise IllegalArgumentException("query and key must be [tokens, heads, headSize]")
        tokens, hq, d = query.shape
        hk = key.shape[1]
        if d != self.head_size or key.shape[2] != d or key.shape[0] != tokens:
            raise IllegalArgumentException("query/key shapes do not match the RoPE head size")
        q_out = torch.empty_like(query)
        k_out = torch.empty_like(key)
        _check(ctx.handle, N.load().nva_rope_forward(
            ctx.handle, self._h, _dev(query, "query"), _dev(key, "key"), tokens, hq, hk,
            _dev(q_out, "q_out"), _dev(k_out, "k_out")), "RotaryEmbedding.forward")
        return q_out, k_out

    def close(self) -> None:
        if self._h:
            N.load().nva_rope_destroy(self._h)
            self._h = None


class RMSNorm:
    """RMSNorm(weight, eps, onePlusWeight) / RMSNorm.weightless(eps) (Norms.java:32-97).

    ``weight`` is a float32 device tensor of the normalised width (kept resident, as the model's
    weights are); ``None`` is the weightless norm."""

    def __init__(self, weight: Optional[torch.Tensor], eps: float,
                 one_plus_weight: bool = False):
        if weight is not None and weight.dim() != 1:
            raise IllegalArgumentException("RMSNorm weight must be 1-D")
        self.weight = weight
        self.eps = float(np.float32(eps))
        self.one_plus_weight = bool(one_plus_weight)
        self._desc = N.RmsNormDesc(None if weight is None else _dev(weight, "weight"), self.eps,
                                   int(self.one_plus_weight))

    @staticmethod
    def weightless(eps: float) -> "RMSNorm":
        return RMSNorm(None, eps)

    def desc(self):
        return ctypes.byref(self._desc)

    def forward(self, x: torch.Tensor, ctx: "Context") -> torch.Tensor:
        """RMSNorm.forward(x): normalises x along its last axis into a new tensor."""
        width = x.shape[-1]
        if self.weight is not None and self.weight.numel() != width:
            raise IllegalArgumentException(
                f"weight has {self.weight.numel()} entries, last dimension is {width}")
        out = torch.empty_like(x)
        rows = x.numel() // width if width else 0
        _check(ctx.handle, N.load().nva_rms_norm_forward(
            ctx.handle, self.desc(), _dev(x, "x"), rows, width, _dev(out, "out")),
            "RMSNorm.forward")
        return out


class Linear:
    """Linear.Row(weight [out, in], bias) (layers/Linear.java:296-335): ``forward(x, ctx)`` is
    Ops.linear, y = x W^T + b, in fp32 on the library's kernels: a GEMV for a few rows, 32 x 32
    blocks for decode batches, 128 x 64 tiles for larger GEMMs.  ``weight``/``bias`` are
    float32 device tensors kept resident, as the model's weights are."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        if weight.dim() != 2:
            raise IllegalArgumentException("weight must be 2D")
        if bias is not None and tuple(bias.shape) != (weight.shape[0],):
            raise IllegalArgumentException("bias must have out entries")
        self.weight = weight
        self.bias = bias
        self.out_features, self.in_features = weight.shape

    def forward(self, x: torch.Tensor, ctx: "Context") -> torch.Tensor:
        if x.numel() % self.in_features != 0:
            raise IllegalArgumentException("x last dim mismatch")
        rows = x.numel() // self.in_features
        y = torch.empty(x.shape[:-1] + (self.out_features,) if x.shape[-1] == self.in_features
                        else (rows, self.out_features), dtype=torch.float32, device=x.device)
        _check(ctx.handle, N.load().nva_linear_forward(
            ctx.handle, _dev(x, "x"), rows, self.in_features, _dev(self.weight, "weight"),
            self.out_features, _dev(self.bias, "bias"), _dev(y, "y")), "Linear.forward")
        return y


class Attention:
    """Attention(numHeads, headDim, scale, numKvHeads, slidingWindow, kvLayerIndex, writeKv)
    (Attention.java:70-125)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int,
                 sliding_window: int = 0, kv_layer_index: int = 0, write_kv: bool = True):
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = float(np.float32(scale))
        self.num_kv_heads = num_kv_heads
        self.sliding_window = max(0, int(sliding_window))
        self.kv_layer_index = kv_layer_index
        self.write_kv = bool(write_kv)
        self._desc = N.AttnDesc(num_heads, head_dim, self.scale, num_kv_heads,
                                self.sliding_window, kv_layer_index, int(self.write_kv))

    def _check_shapes(self, q, k, v) -> None:
        if q.dim() != 3 or tuple(q.shape[1:]) != (self.num_heads, self.head_dim):
            raise IllegalArgumentException(
                f"q must be [tokens, {self.num_heads}, {self.head_dim}], got {tuple(q.shape)}")
        for name, t in (("k", k), ("v", v)):
            if t is not None and tuple(t.shape) != (q.shape[0], self.num_kv_heads, self.head_dim):
                raise IllegalArgumentException(
                    f"{name} must be [{q.shape[0]}, {self.num_kv_heads}, {self.head_dim}], "
                    f"got {tuple(t.shape)}")

    def forward(self, q: torch.Tensor, k: Optional[torch.Tensor], v: Optional[torch.Tensor],
                ctx: Context) -> torch.Tensor:
        """Attention.forward(q, k, v, ctx) (Attention.java:152-171): stores k/v into the bound
        arena at the step's slots, then attends; returns a new [tokens, numHeads, headDim]."""
        self._check_shapes(q, k, v)
        arena = ctx.kv_cache()
        out = torch.empty((q.shape[0], self.num_heads, self.head_dim), dtype=torch.float32,
                          device=q.device)
        _check(ctx.handle, N.load().nva_attention_forward(
            ctx.handle, arena.handle if arena is not None else None, ctypes.byref(self._desc),
            _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), q.shape[0], _dev(out, "out")),
            "Attention.forward")
        return out

    def forward_with_rope(self, rope: RotaryEmbedding, positions, q: torch.Tensor,
                          k: torch.Tensor, v: torch.Tensor, ctx: Context,
                          q_out: Optional[torch.Tensor] = None,
                          k_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """RotaryEmbedding.forward + Attention.forward in one call (the fused RoPE + store
        kernel, then attention), as Qwen3Attention.forward uses them
        (models/internal/Qwen3ForCausalLM.java:207-222)."""
        self._check_shapes(q, k, v)
        for t, shape in ((q_out, q.shape), (k_out, k.shape)):
            if t is not None and tuple(t.shape) != tuple(shape):
                raise IllegalArgumentException("q_out/k_out must match q/k")
        if positions is not None:
            ctx.set_positions(positions)
        arena = ctx.kv_cache()
        out = torch.empty((q.shape[0], self.num_heads, self.head_dim), dtype=torch.float32,
                          device=q.device)
        _check(ctx.handle, N.load().nva_rope_attention_forward(
            ctx.handle, arena.handle if arena is not None else None, rope.handle,
            ctypes.byref(self._desc), _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), q.shape[0],
            _dev(q_out, "q_out"), _dev(k_out, "k_out"), _dev(out, "out")),
            "Attention.forward_with_rope")
        return out

    def forward_with_norm_rope(self, rope: RotaryEmbedding, positions, q: torch.Tensor,
                               k: torch.Tensor, v: torch.Tensor, ctx: Context,
                               q_norm: Optional[RMSNorm] = None,
                               k_norm: Optional[RMSNorm] = None,
                               v_norm: Optional[RMSNorm] = None,
                               q_out: Optional[torch.Tensor] = None,
                               k_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """normHeads(q, qNorm), normHeads(k, kNorm) [, vNorm(v)], RotaryEmbedding.forward and
        Attention.forward as one call (Qwen3ForCausalLM.java:207-227, Gemma3ForCausalLM.java:
        143-157, Gemma4ForCausalLM.java:164-197): one fused kernel normalises, rotates and
        stores, then the attention kernels run."""
        self._check_shapes(q, k, v)
        for t, shape in ((q_out, q.shape), (k_out, k.shape)):
            if t is not None and tuple(t.shape) != tuple(shape):
                raise IllegalArgumentException("q_out/k_out must match q/k")
        for n in (q_norm, k_norm, v_norm):
            if n is not None and n.weight is not None and n.weight.numel() != self.head_dim:
                raise IllegalArgumentException("head norm weights must have headDim entries")
        if positions is not None:
            ctx.set_positions(positions)
        arena = ctx.kv_cache()
        out = torch.empty((q.shape[0], self.num_heads, self.head_dim), dtype=torch.float32,
                          device=q.device)
        _check(ctx.handle, N.load().nva_norm_rope_attention_forward(
            ctx.handle, arena.handle if arena is not None else None, rope.handle,
            None if q_norm is None else q_norm.desc(), None if k_norm is None else k_norm.desc(),
            None if v_norm is None else v_norm.desc(), ctypes.byref(self._desc), _dev(q, "q"),
            _dev(k, "k"), _dev(v, "v"), q.shape[0], _dev(q_out, "q_out"), _dev(k_out, "k_out"),
            _dev(out, "out")), "Attention.forward (q/k norm + RoPE)")
        return out

    def forward_packed_qkv(self, rope: RotaryEmbedding, positions, qkv: torch.Tensor,
                           ctx: Context, q_norm: Optional[RMSNorm] = None,
                           k_norm: Optional[RMSNorm] = None, v_norm: Optional[RMSNorm] = None,
                           q_out: Optional[torch.Tensor] = None,
                           k_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """forward_with_norm_rope on the packed qkv_proj output [T, (Hq + 2 Hkv) * d] (q heads,
        k heads, v heads per token), read in place instead of split by Ops.splitLast
        (Qwen3ForCausalLM.java:210-214)."""
        width = (self.num_heads + 2 * self.num_kv_heads) * self.head_dim
        if qkv.dim() != 2 or qkv.shape[1] != width:
            raise IllegalArgumentException(f"qkv must be [T, {width}]")
        if qkv.dtype != torch.float32 or not qkv.is_contiguous():
            raise IllegalArgumentException("qkv must be a contiguous float32 tensor")
        T = qkv.shape[0]
        for t, shape in ((q_out, (T, self.num_heads, self.head_dim)),
                         (k_out, (T, self.num_kv_heads, self.head_dim))):
            if t is not None and tuple(t.shape) != shape:
                raise IllegalArgumentException("q_out/k_out must be [T, heads, headDim]")
        for n in (q_norm, k_norm, v_norm):
            if n is not None and n.weight is not None and n.weight.numel() != self.head_dim:
                raise IllegalArgumentException("head norm weights must have headDim entries")
        if positions is not None:
            ctx.set_positions(positions)
        arena = ctx.kv_cache()
        out = torch.empty((T, self.num_heads, self.head_dim), dtype=torch.float32,
                          device=qkv.device)
        _check(ctx.handle, N.load().nva_qkv_norm_rope_attention_forward(
            ctx.handle, arena.handle if arena is not None else None, rope.handle,
            None if q_norm is None else q_norm.desc(), None if k_norm is None else k_norm.desc(),
            None if v_norm is None else v_norm.desc(), ctypes.byref(self._desc),
            _dev(qkv, "qkv"), T, _dev(q_out, "q_out"), _dev(k_out, "k_out"), _dev(out, "out")),
            "Attention.forward (packed qkv)")
        return out
