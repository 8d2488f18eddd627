"""Step-metadata producers of libnva.so (include/nva.h: nva_build_prefill_metadata,
nva_build_decode_metadata) over the engine's scheduled sequences.

They restate Transformer.preparePrefill / prepareDecode (engine/Transformer.java:319-456) in the
library's C++ host code, so a model runner hands the scheduled sequences over once per step.
The builders are host-only and need no GPU; ``Context.prepare_prefill`` / ``prepare_decode``
build and upload in one call.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from . import _native as N


@dataclass
class StepMeta:
    """Arguments of Context.set plus the step's positions (Transformer.java:342-457)."""

    is_prefill: bool
    cu_seqlens_q: Optional[np.ndarray]
    cu_seqlens_k: Optional[np.ndarray]
    max_seqlen_q: int
    max_seqlen_k: int
    slot_mapping: Optional[np.ndarray]
    context_lens: Optional[np.ndarray]
    block_tables: Optional[np.ndarray]
    seq_ids: np.ndarray
    positions: np.ndarray

    def context_args(self) -> dict:
        return dict(is_prefill=self.is_prefill, cu_seqlens_q=self.cu_seqlens_q,
                    cu_seqlens_k=self.cu_seqlens_k, max_seqlen_q=self.max_seqlen_q,
                    max_seqlen_k=self.max_seqlen_k, slot_mapping=self.slot_mapping,
                    context_lens=self.context_lens, block_tables=self.block_tables,
                    seq_ids=self.seq_ids, positions=self.positions)


class MetadataError(ValueError):
    """A step the reference's producers would reject (IndexOutOfBounds / NoSuchElement)."""


def seq_array(seqs: Sequence) -> tuple:
    """nva_seq[] for ``seqs`` (objects with seq_id, num_tokens, num_cached_tokens,
    num_scheduled_tokens and block_table, as engine/Sequence.java); the second item keeps the
    block-table arrays alive while the first is in use."""
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
    """nva_build_prefill_metadata (Transformer.preparePrefill) over Sequence-like objects."""
    return _build(seqs, block_size, True)


def build_decode_metadata(seqs, block_size: int) -> StepMeta:
    """nva_build_decode_metadata (Transformer.prepareDecode) over Sequence-like objects."""
    return _build(seqs, block_size, False)
