"""Synthetic single-layer attention workloads at the shapes the benchmark and tests use.

Conventions (shared by every workload):
* numpy ``default_rng(seed)``; context lengths uniform ``rng.integers(lo, hi + 1)`` or
  log-uniform ``floor(exp(rng.uniform(ln lo, ln hi)))``;
* KV block size 256 (the reference's default, llm/Config.java:285);
* block tables are a seeded random permutation of a free pool of ceil(1.25 * pages) blocks,
  capped at 8191 blocks (the most a Java int numel allows at Hkv=8, d=128), handed out to the
  sequences in order;
* a sequence is (cached tokens, new tokens): cached tokens are already in the pages before the
  step, new tokens are stored by the step at their slots (Transformer.java:342-457 metadata).

Named workloads (q heads / kv heads / head dim):
* ``qwen3_decode_small``  Qwen3-0.6B decode, 8 seqs, ctx U[256,1024], 16/8/128.
* ``qwen3_prefill``       Qwen3-0.6B varlen prefill 512/1024/1536/2048, seq 3 has its first
                          1024 tokens (4 full pages) cached, RoPE theta 1e6, 16/8/128.
* ``gemma3_decode``       Gemma3-270M decode, 32 seqs, ctx log-U[512,8192], 4/1/256, scale
                          1/16, local layer window 512 or global layer.
* ``gemma3_prefill``      Gemma3-270M varlen prefill 512/1024/1536/2048, 4/1/256, local or global.
* ``qwen3_decode_large``  Qwen3-0.6B shape decode, 256 seqs, ctx log-U[128,32768].
* ``qwen3_4b_mixed``      Qwen3-4B-like mixed step, 32/8/128: 4 prefill chunks of 512 tokens
                          with prior context U[0,4096] plus 64 decode rows (qLen 1) with ctx
                          U[4096,16384], all in one prefill-with-cache launch.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

from .step import StepMeta

BLOCK_SIZE = 256
POOL_CAP = 8191
QWEN_SCALE = float(np.float32(128.0 ** -0.5))   # (float) Math.pow(128, -0.5)
GEMMA_SCALE = float(np.float32(256.0 ** -0.5))  # query_pre_attn_scalar 256 -> 0.0625


@dataclass
class Workload:
    name: str
    hq: int
    hkv: int
    d: int
    scale: float
    window: int
    block_size: int
    num_blocks: int
    seqs: List[Tuple[int, int]]          # (cached tokens, new tokens) per sequence
    tables: Optional[List[List[int]]]    # block ids per sequence, or None (dense prefill)
    meta: StepMeta
    rope_theta: float = 1e6
    max_pos: int = 40960

    @property
    def tokens(self) -> int:
        return int(sum(n for _, n in self.seqs))

    def slot(self, b: int, t: int) -> int:
        bs = self.block_size
        return self.tables[b][t // bs] * bs + t % bs

    def prior_slots(self) -> np.ndarray:
        """Slots of every cached (pre-step) token."""
        out = [self.slot(b, t) for b, (c, _) in enumerate(self.seqs) for t in range(c)]
        return np.asarray(out, np.int64)

    def kv_bytes_read(self) -> int:
        """Algorithmic K+V bytes attended (each KV head read once per query row)."""
        total = 0
        for c, n in self.seqs:
            for qi in range(n):
                k_len = c + qi + 1
                vis = min(k_len, self.window) if self.window > 0 else k_len
                total += vis
        return total * self.hkv * self.d * 4 * 2

    def visible_pairs(self) -> int:
        """Unmasked (query, key) pairs per query head."""
        total = 0
        for c, n in self.seqs:
            k = np.arange(c + 1, c + n + 1, dtype=np.int64)
            total += int(np.minimum(k, self.window).sum() if self.window > 0 else k.sum())
        return total


def uniform_lengths(rng, n, lo, hi) -> List[int]:
    return [int(x) for x in rng.integers(lo, hi + 1, size=n)]


def loguniform_lengths(rng, n, lo, hi) -> List[int]:
    return [int(math.floor(math.exp(x))) for x in rng.uniform(math.log(lo), math.log(hi), size=n)]


def build(name, seqs, *, is_prefill, hq, hkv, d, scale, window=0, rng=None, paged=True,
          block_size=BLOCK_SIZE, pool_cap=POOL_CAP, rope_theta=1e6, max_pos=40960) -> Workload:
    """Pages, slots, cu_seqlens and positions for ``seqs`` = [(cached, new), ...]."""
    rng = rng if rng is not None else np.random.default_rng(0)
    tables = None
    num_blocks = 1
    if paged:
        pages = [-(-(c + n) // block_size) for c, n in seqs]
        total = sum(pages)
        pool = min(pool_cap, max(1, math.ceil(1.25 * total)))
        if pool < total:
            raise ValueError(f"{total} pages do not fit a pool capped at {pool_cap}")
        perm = rng.permutation(pool)
        tables, at = [], 0
        for p in pages:
            tables.append([int(x) for x in perm[at:at + p]])
            at += p
        num_blocks = pool
    positions, slots, ids = [], [], []
    cu_q, cu_k, lens = [0], [0], []
    for b, (c, n) in enumerate(seqs):
        for t in range(c, c + n):
            positions.append(t)
            ids.append(b)
            if paged:
                slots.append(tables[b][t // block_size] * block_size + t % block_size)
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + c + n)
        lens.append(c + n)
    bt = None
    if paged:
        width = max(len(t) for t in tables)
        bt = np.full((len(seqs), width), -1, np.int32)
        for i, t in enumerate(tables):
            bt[i, :len(t)] = t
    if is_prefill:
        meta = StepMeta(True, np.asarray(cu_q, np.int32), np.asarray(cu_k, np.int32),
                        max(n for _, n in seqs), max(c + n for c, n in seqs),
                        np.asarray(slots, np.int32) if paged else None, None, bt,
                        np.asarray(ids, np.int32), np.asarray(positions, np.float32))
    else:
        assert all(n == 1 for _, n in seqs)
        meta = StepMeta(False, None, None, 0, 0, np.asarray(slots, np.int32),
                        np.asarray(lens, np.int32), bt, np.asarray(ids, np.int32),
                        np.asarray(positions, np.float32))
    return Workload(name, hq, hkv, d, float(np.float32(scale)), window, block_size, num_blocks,
                    list(seqs), tables, meta, rope_theta, max_pos)


def qwen3_decode_small(seed=0) -> Workload:
    rng = np.random.default_rng(seed)
    ctx = uniform_lengths(rng, 8, 256, 1024)
    return build("qwen3-0.6b decode B=8 ctx U[256,1024]", [(c - 1, 1) for c in ctx],
                 is_prefill=False, hq=16, hkv=8, d=128, scale=QWEN_SCALE, rng=rng)


def qwen3_prefill(seed=0) -> Workload:
    rng = np.random.default_rng(seed)
    seqs = [(0, 512), (0, 1024), (0, 1536), (1024, 1024)]
    return build("qwen3-0.6b varlen prefill 512/1024/1536/2048 (seq 3: 1024 cached)", seqs,
                 is_prefill=True, hq=16, hkv=8, d=128, scale=QWEN_SCALE, rng=rng,
                 rope_theta=1e6, max_pos=40960)


def gemma3_decode(seed=0, local=True) -> Workload:
    rng = np.random.default_rng(seed)
    ctx = loguniform_lengths(rng, 32, 512, 8192)
    return build(f"gemma3-270m decode B=32 ctx log-U[512,8192] {'local W=512' if local else 'global'}",
                 [(c - 1, 1) for c in ctx], is_prefill=False, hq=4, hkv=1, d=256,
                 scale=GEMMA_SCALE, window=512 if local else 0, rng=rng,
                 rope_theta=1e4 if local else 1e6, max_pos=32768)


def gemma3_prefill(seed=0, local=True) -> Workload:
    """Gemma3-270M-shaped varlen prefill 512/1024/1536/2048 (no cached prefix), 4/1/256."""
    rng = np.random.default_rng(seed)
    return build(f"gemma3-270m varlen prefill 512/1024/1536/2048 {'local W=512' if local else 'global'}",
                 [(0, 512), (0, 1024), (0, 1536), (0, 2048)], is_prefill=True, hq=4, hkv=1,
                 d=256, scale=GEMMA_SCALE, window=512 if local else 0, rng=rng,
                 rope_theta=1e4 if local else 1e6, max_pos=32768)


def gemma4_prefill_global(seed=0) -> Workload:
    """Gemma-4-text-shaped global (full-attention) layer, varlen prefill 512/1024/1536/2048:
    8 q heads / 1 kv head, head dim 512 (global_head_dim), scale 1.0 (Config.attentionScale:
    q/k are RMS-normed), no window (ModelSupportTest.java:101-118 text_config)."""
    rng = np.random.default_rng(seed)
    return build("gemma4-text global layer varlen prefill 512/1024/1536/2048 (8q/1kv, d=512)",
                 [(0, 512), (0, 1024), (0, 1536), (0, 2048)], is_prefill=True, hq=8, hkv=1,
                 d=512, scale=1.0, window=0, rng=rng, rope_theta=1e6, max_pos=32768)


def gemma4_decode_global(seed=0, batch=32, lo=512, hi=8192) -> Workload:
    """The Gemma-4-text global layer's shape (8 q heads / 1 kv head, head dim 512, scale 1.0)
    in a decode step of ``batch`` rows with log-uniform contexts in [lo, hi]."""
    rng = np.random.default_rng(seed)
    ctx = loguniform_lengths(rng, batch, lo, hi)
    return build(f"gemma4-text global layer decode B={batch} ctx log-U[{lo},{hi}] (8q/1kv, d=512)",
                 [(c - 1, 1) for c in ctx], is_prefill=False, hq=8, hkv=1, d=512, scale=1.0,
                 window=0, rng=rng, rope_theta=1e6, max_pos=32768)


def qwen3_decode_large(seed=0, batch=256, lo=128, hi=32768) -> Workload:
    rng = np.random.default_rng(seed)
    ctx = loguniform_lengths(rng, batch, lo, hi)
    return build(f"qwen3-0.6b decode B={batch} ctx log-U[{lo},{hi}]", [(c - 1, 1) for c in ctx],
                 is_prefill=False, hq=16, hkv=8, d=128, scale=QWEN_SCALE, rng=rng)


def qwen3_decode_large_heads(hq, hkv=8, seed=0, batch=256, lo=128, hi=32768) -> Workload:
    """The headline decode's rows and contexts with another head shape (e.g. Qwen3-14B's 40
    query heads over 8 KV heads, a GQA ratio of 5)."""
    rng = np.random.default_rng(seed)
    ctx = loguniform_lengths(rng, batch, lo, hi)
    return build(f"decode B={batch} ctx log-U[{lo},{hi}], {hq} q heads / {hkv} KV heads, d=128",
                 [(c - 1, 1) for c in ctx], is_prefill=False, hq=hq, hkv=hkv, d=128,
                 scale=QWEN_SCALE, rng=rng)


def qwen3_decode_large_share(ways=8, by="head", seed=0, batch=256, lo=128, hi=32768) -> Workload:
    """One GPU's share of the headline decode sharded ``ways`` ways with no exchange: by KV
    head (all rows, 16/ways q heads over 8/ways KV heads) or by sequence (every ways-th row,
    all heads).  Same contexts as qwen3_decode_large."""
    rng = np.random.default_rng(seed)
    ctx = loguniform_lengths(rng, batch, lo, hi)
    if by == "head":
        return build(f"qwen3-0.6b decode B={batch} ctx log-U[{lo},{hi}], 1/{ways} of the KV heads",
                     [(c - 1, 1) for c in ctx], is_prefill=False, hq=16 // ways, hkv=8 // ways,
                     d=128, scale=QWEN_SCALE, rng=rng)
    rows = ctx[::ways]
    return build(f"qwen3-0.6b decode ctx log-U[{lo},{hi}], every {ways}th of {batch} rows",
                 [(c - 1, 1) for c in rows], is_prefill=False, hq=16, hkv=8, d=128,
                 scale=QWEN_SCALE, rng=rng)


def qwen3_4b_mixed(seed=0, chunks=4, chunk=512, prior_hi=4096, rows=64, ctx_lo=4096,
                   ctx_hi=16384, part="both") -> Workload:
    """The mixed step; part="rows" keeps only its decode rows (a decode step), part="chunks"
    only its prefill chunks (a prefill step), with the same draws."""
    rng = np.random.default_rng(seed)
    prior = uniform_lengths(rng, chunks, 0, prior_hi)
    dec = uniform_lengths(rng, rows, ctx_lo, ctx_hi)
    if part == "rows":
        return build(f"qwen3-4b-like mixed step, its {rows} decode rows alone",
                     [(c - 1, 1) for c in dec], is_prefill=False, hq=32, hkv=8, d=128,
                     scale=QWEN_SCALE, rng=rng)
    if part == "chunks":
        return build(f"qwen3-4b-like mixed step, its {chunks}x{chunk} prefill chunks alone",
                     [(p, chunk) for p in prior], is_prefill=True, hq=32, hkv=8, d=128,
                     scale=QWEN_SCALE, rng=rng)
    seqs = [(p, chunk) for p in prior] + [(c - 1, 1) for c in dec]
    return build(f"qwen3-4b-like mixed: {chunks}x{chunk} prefill chunks (prior U[0,{prior_hi}]) "
                 f"+ {rows} decode rows ctx U[{ctx_lo},{ctx_hi}]", seqs, is_prefill=True, hq=32,
                 hkv=8, d=128, scale=QWEN_SCALE, rng=rng)
