"""CPU oracle for the nano-vllm-java paged-attention path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, by ``__graft_entry__.smoke()`` and by the CPU
baseline leg of ``bench.py``, always as the checker (or the timed CPU baseline), never as part of
the product path.  The product library (``libnva.so``) neither links nor calls anything here.

Two independent restatements live here:

* ``liboracle.so`` (``oracle.c``): the reference's fp32 algorithm restated step by step
  (``Attention.attendJobs`` tile-64 online softmax with ``exp`` in double, the
  ``RotaryEmbedding`` table and apply step, ``storeKvCache``, the ``Attention.forward``
  dispatch).  Citations are in ``oracle.c``.
* ``attention_fp64`` / ``rope_fp64`` below: textbook float64 softmax attention and rotation,
  written from the mathematics with no tiles and no online rescaling.

How each oracle function is pinned (the tests named here live in ``tests/test_oracle.py``):

* ``java_round`` -- against Python's exact ``math.floor(x + 0.5)`` on the float32 grid, including
  halves, negative halves and NaN.
* ``rope_inv_freq`` / ``rope_table`` -- against ``math.pow``/``math.cos``/``math.sin`` evaluated
  in Python doubles with the same float32 casts (IEEE-754 basic ops; libm ``cos``/``sin``/``pow``
  are within 1 ulp of Java's, so a float32 cast can differ only when the double result lies
  within 1 ulp of a float32 rounding boundary -- the Java table itself is uploaded in the real
  integration, so the table bits are identical by construction there).  Closed forms:
  position 0 gives cos=1, sin=0 exactly.
* ``rope_forward`` -- bit-exact against a float32 numpy restatement (numpy float32 ops are
  separately rounded IEEE ops), against the float64 rotation within 1e-6, against the
  pair-norm invariant, and position 0 is the identity.  The planted sign mistake fails.
* ``attention_forward`` -- against ``attention_fp64`` (independent textbook form) within
  1e-5 over random GQA/MQA/window/prefix cases, and against special cases whose answer is
  known in closed form: one visible key gives v; identical keys give the mean of the
  visible V rows; window 1 gives v at the query's own position; MHA equals GQA with
  duplicated K/V; a window >= context equals no window; a qLen=1 prefill-with-cache equals
  decode; negative slots are never written.  Each planted mistake (dropped scale, kvh
  modulo, causal off-by-one, window off-by-one, missing rescale) fails at least one check.
  The reference's own attention tests pin only parallel-vs-sequential self-consistency
  (T/CoreUnitTest.java:1462-1471); that test is re-expressed here too (threads 1 vs 2 must be
  bit-identical).
* ``sum_squares`` / ``rms_norm`` -- ``tests/test_oracle_norm.py``: against the float64 textbook
  ``rms_norm_fp64`` within 2e-6 relative over widths 4..1024 (weightless, weight, onePlusWeight);
  a hand-derived known answer that fixes the scalar summation order ([4096, 1, 1, 1] sums to
  exactly 2^24 because each +1 is a round-to-even tie, while a pairwise tree gives 2^24 + 2);
  exact scale invariance (norm(2x) == norm(x) bit for bit with eps = 0); and the reference's
  own tests re-expressed (T/CoreUnitTest.java:332-349 rows [1.5,1.5] and [4,4] normalise to 1;
  :1047-1056 onePlusWeight equals the plain norm times (1 + w); :675 scalar and vector
  sumSquares of 0.1*i agree within 1e-3).  Planted mistakes (no eps, divide by n - 1,
  pairwise order, onePlusWeight ignored) each fail one of them.
* ``linear`` -- ``tests/test_oracle_linear.py``: against float64 ``x @ W.T + b`` within the
  first-order bound of a sequential fp32 sum ((in + 1) * 2^-24 * sum|terms|), and the reference's own tests re-expressed (T/CoreUnitTest.java:296-300 identity
  weight; :432-471 the sequential sum of x[i]*w[o,i] within 1e-4; :473-502 and :705-728 with a
  bias, scalar vs vector gemv within 1e-4).  Planted mistakes (transposed weight, dropped bias)
  each fail.
* ``store_kv`` -- closed form: ``cache[slot] == k[i]`` for slot >= 0, untouched elsewhere.

Not pinned: the exact bits of Java's ``Math.exp`` and of ``FloatVector.reduceLanes`` (the
JDK leaves the reduction order unspecified and the lane count is host dependent).  These sit
below the path's 1e-4 / 1e-5 tolerance and are bounded by the fp64 comparison above.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

ORC_OK = 0
ORC_E_ARG = -1
ORC_E_ROPE_POS = -2
ORC_E_SHARED_KV = -3
ORC_E_NO_ARENA = -4

MUT_NONE = 0
MUT_DROP_SCALE = 1
MUT_KVH_MODULO = 2
MUT_CAUSAL_OFF1 = 3
MUT_WINDOW_OFF1 = 4
MUT_NO_RESCALE = 5
MUT_ROPE_SIGN = 6
MUT_NORM_NO_EPS = 7
MUT_NORM_DIV_N1 = 8
MUT_NORM_PAIRWISE = 9
MUT_NORM_NO_ONE = 10
MUT_LIN_TRANSPOSE = 11
MUT_LIN_NO_BIAS = 12


class _Attn(ctypes.Structure):
    _fields_ = [
        ("num_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("num_kv_heads", ctypes.c_int),
        ("sliding_window", ctypes.c_int),
        ("write_kv", ctypes.c_int),
    ]


class _Ctx(ctypes.Structure):
    _fields_ = [
        ("is_prefill", ctypes.c_int),
        ("cu_q", ctypes.c_void_p),
        ("cu_k", ctypes.c_void_p),
        ("num_seqs", ctypes.c_int),
        ("slot_mapping", ctypes.c_void_p),
        ("num_slots", ctypes.c_int),
        ("context_lens", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int),
    ]


def build() -> None:
    """Compile liboracle.so from oracle.c (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def build_native(out_path: str) -> str:
    """Compile the same oracle.c for this host (-O3 -march=native) to ``out_path``: the
    benchmark's CPU baseline, built on the machine it is timed on."""
    subprocess.run(["make", "-s", "-C", _HERE, "native", f"NATIVE_OUT={out_path}"], check=True)
    return out_path


def set_library(path: str) -> None:
    """Use the oracle library at ``path`` (e.g. a build_native() build) for every later call."""
    global _lib, _LIB_PATH
    _LIB_PATH = path
    _lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, ci, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.orc_java_round_f32.argtypes = [cf]
        L.orc_java_round_f32.restype = ci
        L.orc_rope_inv_freq.argtypes = [ci, ci, cf, vp]
        L.orc_rope_inv_freq.restype = ci
        L.orc_rope_table.argtypes = [ci, ci, vp, vp]
        L.orc_rope_table.restype = None
        L.orc_rope_forward.argtypes = [vp, ci, ci, vp, vp, vp, vp, vp, ci, ci, ci, ci]
        L.orc_rope_forward.restype = ci
        L.orc_linear.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, ci]
        L.orc_linear.restype = None
        L.orc_sum_squares.argtypes = [vp, ci, ci, ci]
        L.orc_sum_squares.restype = cf
        L.orc_rms_norm.argtypes = [vp, ci, ci, vp, cf, ci, ci, ci, vp]
        L.orc_rms_norm.restype = None
        L.orc_store_kv.argtypes = [vp, vp, vp, ci, ci, vp, vp]
        L.orc_store_kv.restype = None
        L.orc_attention_forward.argtypes = [
            ctypes.POINTER(_Attn), ctypes.POINTER(_Ctx), ci, vp, vp, ci, vp, vp, vp, ci, vp,
            ci, ci, ci]
        L.orc_attention_forward.restype = ci
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> Optional[np.ndarray]:
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


# ------------------------------------------------------------------------------------------ RoPE

def java_round(x: float) -> int:
    return lib().orc_java_round_f32(float(np.float32(x)))


def rope_inv_freq(head_size: int, rotary_dim: int, base: float) -> np.ndarray:
    out = np.zeros(head_size // 2, np.float32)
    rc = lib().orc_rope_inv_freq(head_size, rotary_dim, float(np.float32(base)), _p(out))
    if rc != ORC_OK:
        raise ValueError("rotaryDim must equal headSize")
    return out


def rope_table(head_size: int, max_pos: int, base: float) -> np.ndarray:
    inv = rope_inv_freq(head_size, head_size, base)
    out = np.zeros((max_pos, head_size), np.float32)
    lib().orc_rope_table(head_size, max_pos, _p(inv), _p(out))
    return out


def rope_forward(table: np.ndarray, positions, q, k, mutation: int = MUT_NONE):
    table = _f32(table)
    positions = _f32(positions)
    q = _f32(q)
    k = _f32(k)
    max_pos, head = table.shape
    qo = np.zeros_like(q)
    ko = np.zeros_like(k)
    rc = lib().orc_rope_forward(_p(table), max_pos, head, _p(positions), _p(q), _p(k), _p(qo),
                                _p(ko), q.shape[0], q.shape[1], k.shape[1], mutation)
    if rc == ORC_E_ROPE_POS:
        raise ValueError("RoPE position out of range")
    return qo, ko


def rope_fp64(table: np.ndarray, positions, x: np.ndarray) -> np.ndarray:
    """Textbook rotate-half in float64 with the given (float32) cos/sin table."""
    pos = np.floor(np.asarray(positions, np.float64) + 0.5).astype(np.int64)
    half = x.shape[-1] // 2
    cs = table.astype(np.float64)[pos]                 # [T, d]
    c = cs[:, None, :half]
    s = cs[:, None, half:]
    x = x.astype(np.float64)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


# --------------------------------------------------------------------------------------- RMSNorm

def sum_squares(a, mode: int = 0, mutation: int = MUT_NONE) -> float:
    """VectorMath.sumSquares with the scalar (mode 0) or Vector API (8/16 lanes) backend."""
    a = _f32(a).reshape(-1)
    return float(np.float32(lib().orc_sum_squares(_p(a), a.size, int(mode), int(mutation))))


def rms_norm(x, weight=None, eps: float = 1e-6, one_plus: bool = False, mode: int = 0,
             mutation: int = MUT_NONE) -> np.ndarray:
    """Ops.rmsNorm over the last axis of x (any leading shape).  mode 0 = scalar kernels
    (ScalarFloatKernels.sumSquares order), 8 or 16 = Vector API lanes."""
    x = _f32(x)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    w = None if weight is None else _f32(weight).reshape(-1)
    if w is not None and w.size != width:
        raise ValueError("weight length must equal the last dimension")
    out = np.zeros_like(x)
    lib().orc_rms_norm(_p(x), rows, width, _p(w), float(np.float32(eps)), int(bool(one_plus)),
                       int(mode), int(mutation), _p(out))
    return out


def rms_norm_fp64(x, weight=None, eps: float = 1e-6, one_plus: bool = False) -> np.ndarray:
    """Textbook x / sqrt(mean(x^2) + eps) * w in float64."""
    x = np.asarray(x, np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + float(np.float32(eps)))
    if weight is not None:
        w = np.asarray(weight, np.float64)
        y = y * (1.0 + w if one_plus else w)
    return y


# ---------------------------------------------------------------------------------------- linear

def linear(x, weight, bias=None, mode: int = 0, mutation: int = MUT_NONE) -> np.ndarray:
    """Ops.linear(x, weight [out, in], bias) on the sequential runtime: x @ weight.T + bias,
    with the scalar (mode 0) or Vector API (8 / 16 lanes) gemv order."""
    x = _f32(x)
    w = _f32(weight)
    out_f, in_f = w.shape
    rows = x.size // in_f
    b = None if bias is None else _f32(bias)
    y = np.zeros(x.shape[:-1] + (out_f,), np.float32)
    lib().orc_linear(_p(x), _p(w), _p(b), _p(y), rows, in_f, out_f, int(mode), int(mutation))
    return y


# ------------------------------------------------------------------------------------- attention

def store_kv(key, value, slots, k_cache: np.ndarray, v_cache: np.ndarray) -> None:
    key = _f32(key)
    value = _f32(value)
    slots = _i32(slots)
    row = key.shape[1] * key.shape[2]
    lib().orc_store_kv(_p(key), _p(value), _p(slots), key.shape[0], row, _p(k_cache), _p(v_cache))


def attention_forward(num_heads, head_dim, scale, num_kv_heads, *, is_prefill, q, k=None, v=None,
                      cu_q=None, cu_k=None, slot_mapping=None, context_lens=None,
                      block_tables=None, k_cache=None, v_cache=None, sliding_window=0,
                      write_kv=True, has_arena=True, threads=1, kernels=0,
                      mutation=MUT_NONE) -> np.ndarray:
    """``Attention.forward`` restated (oracle.c).  ``k_cache``/``v_cache`` are
    ``[num_blocks, block_size, Hkv, d]`` float32 arrays mutated in place (the store), or None
    for a layer whose arena tensor is the numel-1 dummy.  ``kernels`` selects the float kernel
    semantics: 0 = ScalarFloatKernels, 8 or 16 = VectorFloatKernels with that lane count."""
    q = _f32(q)
    T = q.shape[0]
    k = _f32(k) if k is not None else np.zeros((T, num_kv_heads, head_dim), np.float32)
    v = _f32(v) if v is not None else np.zeros((T, num_kv_heads, head_dim), np.float32)
    a = _Attn(num_heads, head_dim, float(np.float32(scale)), num_kv_heads,
              max(0, int(sliding_window)), int(bool(write_kv)))
    cu_q, cu_k = _i32(cu_q), _i32(cu_k)
    slots = _i32(slot_mapping)
    ctx_lens = _i32(context_lens)
    bt = _i32(block_tables)
    if bt is not None and bt.ndim == 2 and bt.shape[1] == 0:
        bt = np.full((bt.shape[0], 1), -1, np.int32)
    c = _Ctx(int(bool(is_prefill)), _p(cu_q), _p(cu_k),
             (len(cu_q) - 1) if cu_q is not None else T,
             _p(slots), len(slots) if slots is not None else 0,
             _p(ctx_lens), _p(bt), bt.shape[1] if bt is not None else 0)
    block_size = 1
    if k_cache is not None:
        assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
        assert v_cache.dtype == np.float32 and v_cache.flags.c_contiguous
        block_size = k_cache.shape[1]
    out = np.zeros((T, num_heads, head_dim), np.float32)
    rc = lib().orc_attention_forward(ctypes.byref(a), ctypes.byref(c), int(bool(has_arena)),
                                     _p(k_cache), _p(v_cache), block_size, _p(q), _p(k), _p(v),
                                     T, _p(out), int(threads), int(kernels), int(mutation))
    if rc == ORC_E_NO_ARENA:
        raise TypeError("KV cache arena not bound in Context")
    if rc == ORC_E_SHARED_KV:
        raise RuntimeError(
            "shared-KV attention needs slot mapping or block tables to read the producer cache")
    if rc != ORC_OK:
        raise ValueError(f"oracle error {rc}")
    return out


def attention_fp64(num_heads, head_dim, scale, num_kv_heads, *, is_prefill, q, k=None, v=None,
                   cu_q=None, cu_k=None, context_lens=None, block_tables=None, k_cache=None,
                   v_cache=None, sliding_window=0) -> np.ndarray:
    """Textbook softmax attention in float64, written from the definition (no tiles, no
    online rescaling).  K/V are taken from the *already stored* cache for the paged cases and
    from dense k/v for the dense prefill case; the caller performs the store first."""
    q = np.asarray(q, np.float64)
    T = q.shape[0]
    rep = num_heads // num_kv_heads
    W = max(0, int(sliding_window))
    out = np.zeros((T, num_heads, head_dim), np.float64)
    sc = float(np.float32(scale))

    def rows_for(b, k_len, paged):
        if paged:
            bs = k_cache.shape[1]
            table = np.asarray(block_tables[b], np.int64)
            j = np.arange(k_len)
            slots = table[j // bs] * bs + j % bs
            kc = k_cache.reshape(-1, num_kv_heads, head_dim)
            vc = v_cache.reshape(-1, num_kv_heads, head_dim)
            return kc[slots].astype(np.float64), vc[slots].astype(np.float64)
        base = int(cu_k[b])
        return (np.asarray(k, np.float64)[base:base + k_len],
                np.asarray(v, np.float64)[base:base + k_len])

    if is_prefill:
        seqs = [(int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b + 1] - cu_k[b]), True)
                for b in range(len(cu_q) - 1)]
        paged = block_tables is not None
    else:
        seqs = [(b, b + 1, int(context_lens[b]), False) for b in range(T)]
        paged = True
    for b, (q0, q1, k_len, causal) in enumerate(seqs):
        q_len = q1 - q0
        if k_len <= 0 or q_len <= 0:
            continue
        K, V = rows_for(b, k_len, paged)
        for qi in range(q_len):
            abs_q = (k_len - q_len + qi) if causal else (k_len - 1)
            end = abs_q + 1 if causal else k_len
            start = max(0, abs_q - W + 1) if W > 0 else 0
            if end <= start:
                continue
            for h in range(num_heads):
                kvh = h // rep
                s = K[start:end, kvh, :] @ q[q0 + qi, h, :] * sc
                w = np.exp(s - s.max())
                out[q0 + qi, h, :] = (w[:, None] * V[start:end, kvh, :]).sum(0) / w.sum()
    return out


def filled_ramp(*shape) -> np.ndarray:
    """T/CoreUnitTest.java:574-584 ``filledRamp``: element i = (i % 17) * 0.1f - 0.8f."""
    n = int(np.prod(shape))
    i = np.arange(n)
    vals = (i % 17).astype(np.float32) * np.float32(0.1) - np.float32(0.8)
    return vals.astype(np.float32).reshape(shape)
