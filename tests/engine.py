"""Host-side producers of the step metadata the attention boundary consumes.

These stay on the engine side of the boundary (in the reference they are Java and are not
replaced); they are restated here, as test infrastructure, so that the tests can drive the
library with exactly the block ids and metadata the reference's engine would hand it:

* ``Sequence``       -- engine/Sequence.java:323-361 (numBlocks, lastBlockNumTokens, block).
* ``BlockManager``   -- engine/BlockManager.java:77-266 (paged allocator, prefix-cache hashing:
                        FNV-1a over little-endian token bytes XOR CRC32(prefix, tokens) * poly).
* ``prepare_prefill`` / ``prepare_decode`` / ``prepare_block_tables`` --
                        engine/Transformer.java:320-457 (cu_seqlens, positions, slot mapping,
                        -1-padded block tables).

(Reference paths are relative to nano-vllm-java/src/main/java/com/igormaznitsa/nanollvm/.)
"""

from __future__ import annotations

import struct
import zlib
from collections import deque
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from nanollvm_amd.step import StepMeta

_MASK64 = (1 << 64) - 1
_FNV_OFFSET = 0xCBF29CE484222325
_FNV_PRIME = 0x100000001B3
_HASH_POLY = 0xC96C5795D7870F42


def _signed64(x: int) -> int:
    x &= _MASK64
    return x - (1 << 64) if x >> 63 else x


class Sequence:
    """The parts of engine/Sequence.java the paging and metadata code reads."""

    _next_id = 0

    def __init__(self, token_ids: List[int], block_size: int):
        self.token_ids = list(token_ids)
        self.block_size = block_size
        self.block_table: List[int] = []
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.seq_id = Sequence._next_id
        Sequence._next_id += 1

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    def length(self) -> int:
        return len(self.token_ids)

    def num_blocks(self) -> int:
        return (self.num_tokens + self.block_size - 1) // self.block_size

    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks() - 1) * self.block_size

    def block(self, i: int) -> List[int]:
        if i < 0 or i >= self.num_blocks():
            raise IndexError(f"block {i}")
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def append_token(self, token: int) -> None:
        self.token_ids.append(token)


@dataclass
class _Block:
    block_id: int
    ref_count: int = 0
    hash: int = -1
    token_ids: List[int] = field(default_factory=list)


class BlockManager:
    """engine/BlockManager.java: free list is a deque (pollFirst / addLast); prefix hits cover only
    leading FULL pages, never the last page."""

    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.blocks = [_Block(i) for i in range(num_blocks)]
        self.hash_to_block: Dict[int, int] = {}
        self.free = deque(range(num_blocks))
        self.used = set()

    @staticmethod
    def compute_hash(token_ids: List[int], prefix: int) -> int:
        """BlockManager.computeHash (BlockManager.java:77-101), as a signed 64-bit value."""
        h = _FNV_OFFSET
        if prefix != -1:
            h = ((h ^ (prefix & _MASK64)) * _FNV_PRIME) & _MASK64
        for tok in token_ids:
            for byte in struct.pack("<i", tok):
                h = ((h ^ byte) * _FNV_PRIME) & _MASK64
        crc = zlib.crc32(struct.pack("<q", prefix) + b"".join(struct.pack("<i", t)
                                                               for t in token_ids))
        return _signed64(h ^ ((crc * _HASH_POLY) & _MASK64))

    def _allocate_block(self) -> int:
        if not self.free:
            raise RuntimeError("no free KV blocks")
        bid = self.free.popleft()
        blk = self.blocks[bid]
        if blk.hash != -1 and self.hash_to_block.get(blk.hash, -1) == bid:
            del self.hash_to_block[blk.hash]
        blk.ref_count = 1
        blk.hash = -1
        blk.token_ids = []
        self.used.add(bid)
        return bid

    def _deallocate_block(self, bid: int) -> None:
        self.used.discard(bid)
        self.free.append(bid)

    def can_allocate(self, seq: Sequence) -> int:
        h = -1
        cached = 0
        new_blocks = seq.num_blocks()
        for i in range(seq.num_blocks() - 1):
            toks = seq.block(i)
            h = self.compute_hash(toks, h)
            bid = self.hash_to_block.get(h, -1)
            if bid == -1 or self.blocks[bid].token_ids != toks:
                break
            cached += 1
            if bid in self.used:
                new_blocks -= 1
        if len(self.free) < new_blocks:
            return -1
        return cached

    def allocate(self, seq: Sequence, num_cached_blocks: int) -> None:
        if seq.block_table:
            raise RuntimeError("sequence already has block table")
        h = -1
        for i in range(num_cached_blocks):
            h = self.compute_hash(seq.block(i), h)
            bid = self.hash_to_block[h]
            blk = self.blocks[bid]
            if bid in self.used:
                blk.ref_count += 1
            else:
                blk.ref_count = 1
                self.free.remove(bid)
                self.used.add(bid)
            seq.block_table.append(bid)
        for _ in range(num_cached_blocks, seq.num_blocks()):
            seq.block_table.append(self._allocate_block())
        seq.num_cached_tokens = num_cached_blocks * self.block_size

    def deallocate(self, seq: Sequence) -> None:
        for bid in reversed(seq.block_table):
            blk = self.blocks[bid]
            blk.ref_count -= 1
            if blk.ref_count == 0:
                self._deallocate_block(bid)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq: Sequence) -> bool:
        return len(self.free) >= (1 if seq.length() % self.block_size == 1 else 0)

    def may_append(self, seq: Sequence) -> None:
        if seq.length() % self.block_size == 1:
            seq.block_table.append(self._allocate_block())

    def hash_blocks(self, seq: Sequence) -> None:
        start = seq.num_cached_tokens // self.block_size
        end = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        if start == end:
            return
        h = self.blocks[seq.block_table[start - 1]].hash if start > 0 else -1
        for i in range(start, end):
            blk = self.blocks[seq.block_table[i]]
            toks = seq.block(i)
            h = self.compute_hash(toks, h)
            blk.hash = h
            blk.token_ids = list(toks)
            self.hash_to_block[h] = blk.block_id


def prepare_block_tables(tables: List[List[int]]) -> np.ndarray:
    """Transformer.prepareBlockTables (Transformer.java:320-331): rectangular, -1 padded."""
    width = max((len(t) for t in tables), default=0)
    out = np.full((len(tables), width), -1, np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = t
    return out


def prepare_prefill(seqs: List[Sequence], block_size: int) -> StepMeta:
    """Transformer.preparePrefill (Transformer.java:342-424)."""
    positions, seq_ids, slots = [], [], []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    any_table = False
    for seq in seqs:
        start = seq.num_cached_tokens
        qlen = seq.num_scheduled_tokens
        end = start + qlen
        positions.extend(range(start, end))
        seq_ids.extend([seq.seq_id] * qlen)
        cu_q.append(cu_q[-1] + qlen)
        cu_k.append(cu_k[-1] + end)
        max_q = max(max_q, qlen)
        max_k = max(max_k, end)
        if not seq.block_table:
            continue
        any_table = True
        sb = start // block_size
        eb = (end + block_size - 1) // block_size
        for i in range(sb, eb):
            s0 = seq.block_table[i] * block_size
            if i == sb:
                s0 += start % block_size
            if i != eb - 1:
                s1 = seq.block_table[i] * block_size + block_size
            else:
                s1 = seq.block_table[i] * block_size + end - i * block_size
            slots.extend(range(s0, s1))
    tables = None
    if cu_k[-1] > cu_q[-1] and any_table:
        tables = prepare_block_tables([s.block_table for s in seqs])
    return StepMeta(True, np.asarray(cu_q, np.int32), np.asarray(cu_k, np.int32), max_q, max_k,
                    np.asarray(slots, np.int32), None, tables, np.asarray(seq_ids, np.int32),
                    np.asarray(positions, np.float32))


def prepare_decode(seqs: List[Sequence], block_size: int) -> StepMeta:
    """Transformer.prepareDecode (Transformer.java:433-457)."""
    n = len(seqs)
    positions = np.zeros(n, np.float32)
    slots = np.zeros(n, np.int32)
    lens = np.zeros(n, np.int32)
    ids = np.zeros(n, np.int32)
    for i, seq in enumerate(seqs):
        positions[i] = seq.length() - 1
        lens[i] = seq.length()
        ids[i] = seq.seq_id
        slots[i] = seq.block_table[-1] * block_size + seq.last_block_num_tokens() - 1
    return StepMeta(False, None, None, 0, 0, slots, lens,
                    prepare_block_tables([s.block_table for s in seqs]), ids, positions)
