"""Step-metadata producers of libnva.so (include/nva.h: nva_build_prefill_metadata,
nva_build_decode_metadata) over the engine's ``Sequence`` objects.

They restate Transformer.preparePrefill / prepareDecode (engine/Transformer.java:319-456) in the
library's C++ host code, so a model runner hands the scheduled sequences over once per step.
The builders are host-only and need no GPU; ``Context.prepare_prefill`` / ``prepare_decode``
build and upload in one call.
"""

from __future__ import annotations

import ctypes
from typing import List, Sequence

import numpy as np

from . import _native as N
from .engine import StepMeta


class MetadataError(ValueError):
    """A step the reference's producers would reject (IndexOutOfBounds / NoSuchElement)."""


def seq_array(seqs: Sequence) -> tuple:
    """nva_seq[] for ``seqs`` (engine.Sequence objects); the second item keeps the block-table
    arrays alive while the first is in use."""
    arr = (N.Seq * max(1, len(seqs)))()
    keep: List[np.ndarray] = []
    for i, s in enumerate(seqs):
        t = np.ascontiguousarray(s.block_table, dtype=np.int32)
        keep.append(t)
        arr[i] = N.Seq(s.seq_id, s.num_tokens, s.num_cached_tokens, s.num_scheduled_tokens,
                       t.ctypes.data if t.size else None, int(t.size))
    return arr, keep


def _build(seqs, block_size: int, prefill: bool) -> StepMeta:
    n = len(seqs)
    tokens = sum(s.num_scheduled_tokens for s in seqs) if prefill else n
    width = max((len(s.block_table) for s in seqs), default=0)
    cu_q = np.zeros(n + 1, np.int32)
    cu_k = np.zeros(n + 1, np.int32)
    slots = np.zeros(max(tokens, 1), np.int32)
    lens = np.zeros(max(n, 1), np.int32)
    ids = np.zeros(max(tokens, 1), np.int32)
    pos = np.zeros(max(tokens, 1), np.float32)
    tables = np.zeros(max(n * width, 1), np.int32)
    out = N.StepMetaOut(cu_q.ctypes.data, cu_k.ctypes.data, 0, 0, slots.ctypes.data, 0,
                        lens.ctypes.data, ids.ctypes.data, pos.ctypes.data, 0,
                        tables.ctypes.data, 0, 0)
    arr, keep = seq_array(seqs)
    fn = N.load().nva_build_prefill_metadata if prefill else N.load().nva_build_decode_metadata
    st = fn(arr, n, block_size, ctypes.byref(out))
    del keep
    if st != N.NVA_OK:
        raise MetadataError(N.load().nva_status_string(st).decode())
    bt = tables[:n * out.bt_stride].reshape(n, out.bt_stride) if out.has_tables else None
    T = out.num_tokens
    if prefill:
        return StepMeta(True, cu_q, cu_k, out.max_seqlen_q, out.max_seqlen_k,
                        slots[:out.num_slots], None, bt, ids[:T], pos[:T])
    return StepMeta(False, None, None, 0, 0, slots[:out.num_slots], lens[:n], bt, ids[:T],
                    pos[:T])


def build_prefill_metadata(seqs, block_size: int) -> StepMeta:
    """nva_build_prefill_metadata (Transformer.preparePrefill) over engine.Sequence objects."""
    return _build(seqs, block_size, True)


def build_decode_metadata(seqs, block_size: int) -> StepMeta:
    """nva_build_decode_metadata (Transformer.prepareDecode) over engine.Sequence objects."""
    return _build(seqs, block_size, False)
