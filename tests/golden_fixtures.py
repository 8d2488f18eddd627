"""Loader for the golden fixtures in ``tests/golden`` (numpy arrays only, loaded without
pickles) and the oracle call that re-derives an attention fixture."""

import glob
import os

import numpy as np

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def names(kind=None):
    out = []
    for p in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        name = os.path.basename(p)[:-4]
        if kind is None or str(load(name)["kind"]) == kind:
            out.append(name)
    return out


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def meta(fx):
    """The fixture's step metadata as Context.set keyword arguments."""
    m = {k[5:]: fx[k] for k in fx if k.startswith("meta_")}
    m["is_prefill"] = bool(m["is_prefill"])
    for k in ("max_seqlen_q", "max_seqlen_k"):
        if k in m:
            m[k] = int(m[k])
    return m


def oracle_attention(fx):
    """Re-runs the oracle on an attention fixture: (out, k_cache_after, v_cache_after)."""
    m = meta(fx)
    kc = fx["k_cache"].copy() if "k_cache" in fx else None
    vc = fx["v_cache"].copy() if "v_cache" in fx else None
    out = O.attention_forward(
        int(fx["hq"]), int(fx["d"]), float(fx["scale"]), int(fx["hkv"]),
        is_prefill=m["is_prefill"], q=fx["q"], k=fx["k"], v=fx["v"], cu_q=m.get("cu_seqlens_q"),
        cu_k=m.get("cu_seqlens_k"), slot_mapping=m.get("slot_mapping"),
        context_lens=m.get("context_lens"), block_tables=m.get("block_tables"), k_cache=kc,
        v_cache=vc, sliding_window=int(fx["window"]))
    return out, kc, vc
