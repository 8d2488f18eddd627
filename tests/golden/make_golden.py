"""Writes the golden fixtures in this folder: small inputs with the oracle's outputs for them.
Every fixture is cross-checked against the float64 closed forms before it is written, so a
fixture is never saved from an oracle that disagrees with the mathematics.

    python tests/golden/make_golden.py        (from the repository root)

Each ``<name>.npz`` holds numpy arrays only (no pickles): the inputs, the step metadata
(``meta_*``, absent fields omitted), scalars as 0-d arrays, and the expected outputs.
``tests/test_golden.py`` re-derives every fixture with the oracle (which must reproduce it bit
for bit) and ``tests/test_gpu_golden.py`` checks the library against it."""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tests"), os.path.join(ROOT, "nano-vllm-java_amd")]

from cases import Case  # noqa: E402
from nanollvm_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

META = ("is_prefill", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k",
        "slot_mapping", "context_lens", "block_tables", "seq_ids", "positions")
ATT_TOL = (1e-5, 1e-6)  # fp32 oracle vs float64: max-abs, rel-L2 at these sizes


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    n = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (n if n > 0 else 1.0))


def meta_arrays(meta) -> dict:
    out = {}
    for f in META:
        val = getattr(meta, f)
        if val is None:
            continue
        if f == "block_tables" and not isinstance(val, np.ndarray):
            width = max((len(t) for t in val), default=0)
            arr = np.full((len(val), width), -1, np.int32)
            for i, t in enumerate(val):
                arr[i, :len(t)] = t
            val = arr
        out["meta_" + f] = np.asarray(val)
    return out


def attention_fixture(name, case: Case, note: str) -> dict:
    wl = case.wl
    out, kc, vc = case.oracle(threads=1)
    ref = case.fp64(kc, vc)
    err, rl2 = float(np.max(np.abs(out - ref))), rel_l2(out, ref)
    assert err <= ATT_TOL[0] and rl2 <= ATT_TOL[1], (name, err, rl2)
    arrays = dict(kind=np.asarray("attention"), note=np.asarray(note), hq=np.int32(wl.hq),
                  hkv=np.int32(wl.hkv), d=np.int32(wl.d), scale=np.float32(wl.scale),
                  window=np.int32(wl.window), q=case.q, k=case.k, v=case.v, out=out,
                  **meta_arrays(wl.meta))
    if case.paged:
        arrays.update(block_size=np.int32(wl.block_size), k_cache=case.k_cache,
                      v_cache=case.v_cache, k_cache_out=kc, v_cache_out=vc)
    print(f"{name}: max-abs vs fp64 {err:.2e}, rel-L2 {rl2:.2e}")
    return arrays


def ref_causal_prefill() -> dict:
    """T/CoreUnitTest.java:1462-1471: Attention(8, 4, 1f, 8), filledRamp q = k = v [16, 8, 4],
    dense prefill over one 16-token sequence, no slots."""
    q = O.filled_ramp(16, 8, 4)
    meta = dict(meta_is_prefill=np.asarray(True), meta_cu_seqlens_q=np.array([0, 16], np.int32),
                meta_cu_seqlens_k=np.array([0, 16], np.int32), meta_max_seqlen_q=np.int32(16),
                meta_max_seqlen_k=np.int32(16))
    out = O.attention_forward(8, 4, 1.0, 8, is_prefill=True, q=q, k=q, v=q, cu_q=[0, 16],
                              cu_k=[0, 16])
    ref = O.attention_fp64(8, 4, 1.0, 8, is_prefill=True, q=q, k=q, v=q, cu_q=[0, 16],
                           cu_k=[0, 16])
    err = float(np.max(np.abs(out - ref)))
    assert err <= 1e-5, err
    print(f"ref_causal_prefill_d4: max-abs vs fp64 {err:.2e}")
    return dict(kind=np.asarray("attention"), note=np.asarray("T/CoreUnitTest.java:1462-1471"),
                hq=np.int32(8), hkv=np.int32(8), d=np.int32(4), scale=np.float32(1.0),
                window=np.int32(0), q=q, k=q, v=q, out=out, **meta)


def ref_rope() -> dict:
    """T/CoreUnitTest.java:1487-1505: RotaryEmbedding(8, 8, 128, 1e4), 64 tokens, 8 q / 4 k
    heads of filledRamp; outputs bit-exact."""
    table = O.rope_table(8, 128, 1e4)
    q, k = O.filled_ramp(64, 8, 8), O.filled_ramp(64, 4, 8)
    pos = np.arange(64, dtype=np.float32)
    qr, kr = O.rope_forward(table, pos, q, k)
    for x, y in ((q, qr), (k, kr)):
        assert np.max(np.abs(O.rope_fp64(table, pos, x) - y)) <= 1e-6
    return dict(kind=np.asarray("rope"), note=np.asarray("T/CoreUnitTest.java:1487-1505"),
                head_size=np.int32(8), max_pos=np.int32(128), base=np.float64(1e4), table=table,
                positions=pos, q=q, k=k, q_out=qr, k_out=kr)


def rms_norm_rows() -> dict:
    rng = np.random.default_rng(2024)
    x = (rng.standard_normal((37, 128)) * 3.0).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    outs = {}
    for tag, weight, one_plus in (("weightless", None, False), ("weight", w, False),
                                  ("one_plus", w, True)):
        y = O.rms_norm(x, weight, 1e-6, one_plus)
        ref = O.rms_norm_fp64(x, weight, 1e-6, one_plus)
        assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) <= 2e-6, tag
        outs["out_" + tag] = y
    return dict(kind=np.asarray("rms_norm"), note=np.asarray("RMSNorm.forward, scalar order"),
                x=x, weight=w, eps=np.float32(1e-6), **outs)


def linear_small() -> dict:
    rng = np.random.default_rng(77)
    x = rng.standard_normal((5, 132)).astype(np.float32)
    w = (rng.standard_normal((72, 132)) / 12.0).astype(np.float32)
    b = rng.standard_normal(72).astype(np.float32)
    y = O.linear(x, w, b)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    bound = 133 * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).T.astype(np.float64)
                                + np.abs(b))
    assert np.all(np.abs(y - ref) <= bound + 1e-7)
    return dict(kind=np.asarray("linear"), note=np.asarray("Linear.Row / Ops.linear"), x=x, w=w,
                b=b, y=y)


def main() -> None:
    fixtures = {
        "ref_causal_prefill_d4": ref_causal_prefill(),
        "ref_rope_d8": ref_rope(),
        "rms_norm_rows": rms_norm_rows(),
        "linear_small": linear_small(),
    }
    rng = np.random.default_rng(11)
    ctx = [1, 2, 15, 16, 17, 40, 63, 64, 65, 100]
    wl = W.build("golden decode gqa", [(c - 1, 1) for c in ctx], is_prefill=False, hq=4, hkv=2,
                 d=16, scale=0.25, rng=rng, block_size=16)
    fixtures["decode_gqa_paged"] = attention_fixture(
        "decode_gqa_paged", Case(wl, seed=5), "decode, GQA 2:1, 16-token pages")
    wl = W.build("golden prefill window", [(20, 30), (0, 17), (3, 40)], is_prefill=True, hq=4,
                 hkv=2, d=32, scale=0.2, window=9, rng=rng, block_size=16)
    fixtures["prefill_paged_window"] = attention_fixture(
        "prefill_paged_window", Case(wl, seed=6),
        "prefill with cache, window 9, prefix hit and mid-page start")
    wl = W.build("golden prefill mfma", [(16, 70), (5, 33), (0, 2), (9, 1)], is_prefill=True,
                 hq=2, hkv=1, d=64, scale=0.125, rng=rng, block_size=16)
    fixtures["prefill_paged_d64"] = attention_fixture(
        "prefill_paged_d64", Case(wl, seed=7),
        "prefill with cache at head dim 64 (MFMA tiles on the GPU), a one-query row")
    for name, arrays in fixtures.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        print(f"wrote {name}.npz ({os.path.getsize(os.path.join(HERE, name + '.npz'))} bytes)")


if __name__ == "__main__":
    main()
