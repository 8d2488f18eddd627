"""ctypes binding of libnva.so (include/nva.h).

The shared library is the product: every compute call goes through it.  There is no Python or
CPU fallback -- loading fails with an ImportError when libnva.so is missing, and creating a
context fails when no HIP device is usable.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnva.so")

NVA_OK = 0
NVA_E_ARG = 1
NVA_E_LAYER = 2
NVA_E_ROPE_POS = 3
NVA_E_SHARED_KV = 4
NVA_E_NO_ARENA = 5
NVA_E_NO_STEP = 6
NVA_E_HIP = 7
NVA_E_OOM = 8
NVA_E_UNSUPPORTED = 9

# Every symbol include/nva.h declares, with its ctypes signature.
_vp = ctypes.c_void_p
_ci = ctypes.c_int
_cf = ctypes.c_float
_i64 = ctypes.c_int64
_st = ctypes.c_int32
_pvp = ctypes.POINTER(ctypes.c_void_p)


class AttnDesc(ctypes.Structure):
    """nva_attn_desc: the arguments of the Attention constructor (Attention.java:108-125)."""

    _fields_ = [
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("num_kv_heads", ctypes.c_int32),
        ("sliding_window", ctypes.c_int32),
        ("kv_layer_index", ctypes.c_int32),
        ("write_kv", ctypes.c_int32),
    ]


class RmsNormDesc(ctypes.Structure):
    """nva_rms_norm: RMSNorm(weight, eps, onePlusWeight) (layers/Norms.java:32-97); weight is a
    device pointer or None (weightless)."""

    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("one_plus_weight", ctypes.c_int32),
    ]


_pnorm = ctypes.POINTER(RmsNormDesc)


class Seq(ctypes.Structure):
    """nva_seq: one scheduled sequence (engine/Sequence.java) with its block table."""

    _fields_ = [
        ("seq_id", ctypes.c_int32),
        ("num_tokens", ctypes.c_int32),
        ("num_cached_tokens", ctypes.c_int32),
        ("num_scheduled", ctypes.c_int32),
        ("block_table", ctypes.c_void_p),
        ("num_blocks", ctypes.c_int32),
    ]


class StepMetaOut(ctypes.Structure):
    """nva_step_meta: caller-owned host arrays the step producers fill."""

    _fields_ = [
        ("cu_q", ctypes.c_void_p),
        ("cu_k", ctypes.c_void_p),
        ("max_seqlen_q", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("slot_mapping", ctypes.c_void_p),
        ("num_slots", ctypes.c_int32),
        ("context_lens", ctypes.c_void_p),
        ("seq_ids", ctypes.c_void_p),
        ("positions", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int32),
        ("block_tables", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int32),
        ("has_tables", ctypes.c_int32),
    ]


_pseq = ctypes.POINTER(Seq)
_pmeta = ctypes.POINTER(StepMetaOut)

SIGNATURES = {
    "nva_ctx_create": ([_ci, _pvp], _st),
    "nva_ctx_destroy": ([_vp], _st),
    "nva_ctx_set_stream": ([_vp, _vp], _st),
    "nva_ctx_stream": ([_vp], _vp),
    "nva_ctx_sync": ([_vp], _st),
    "nva_last_error": ([_vp], ctypes.c_char_p),
    "nva_status_string": ([_st], ctypes.c_char_p),
    "nva_ctx_set_timing": ([_vp, _ci], _st),
    "nva_ctx_kernel_stats": ([_vp, ctypes.c_char_p, ctypes.POINTER(_i64),
                              ctypes.POINTER(ctypes.c_double)], _st),
    "nva_ctx_reset_stats": ([_vp], _st),
    "nva_kv_create": ([_vp, _ci, _ci, _ci, _ci, _vp, _vp, _pvp], _st),
    "nva_kv_destroy": ([_vp], _st),
    "nva_kv_blocks_that_fit": ([_vp, _ci, _ci, _ci, _vp, _vp, _cf, ctypes.POINTER(_ci),
                                ctypes.POINTER(_i64)], _st),
    "nva_kv_layer": ([_vp, _ci, _pvp, _pvp, ctypes.POINTER(_i64)], _st),
    "nva_kv_write": ([_vp, _ci, _ci, _i64, _vp, _i64], _st),
    "nva_kv_read": ([_vp, _ci, _ci, _i64, _vp, _i64], _st),
    "nva_rope_create": ([_vp, _vp, _ci, _ci, _pvp], _st),
    "nva_rope_create_theta": ([_vp, _ci, _ci, _ci, _cf, _pvp], _st),
    "nva_rope_destroy": ([_vp], _st),
    "nva_step_set": ([_vp, _ci, _vp, _vp, _ci, _ci, _ci, _vp, _ci, _vp, _vp, _ci, _vp, _vp, _ci],
                     _st),
    "nva_step_positions": ([_vp, _vp, _ci], _st),
    "nva_step_clear": ([_vp], _st),
    "nva_rope_forward": ([_vp, _vp, _vp, _vp, _ci, _ci, _ci, _vp, _vp], _st),
    "nva_attention_forward": ([_vp, _vp, ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _ci, _vp], _st),
    "nva_attention_forward_noalloc": ([_vp, _vp, ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _ci,
                                       _vp], _st),
    "nva_rope_attention_forward": ([_vp, _vp, _vp, ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _ci,
                                    _vp, _vp, _vp], _st),
    "nva_rms_norm_forward": ([_vp, _pnorm, _vp, _ci, _ci, _vp], _st),
    "nva_linear_forward": ([_vp, _vp, _ci, _ci, _vp, _ci, _vp, _vp], _st),
    "nva_build_prefill_metadata": ([_pseq, _ci, _ci, _pmeta], _st),
    "nva_build_decode_metadata": ([_pseq, _ci, _ci, _pmeta], _st),
    "nva_step_prepare_prefill": ([_vp, _pseq, _ci, _ci], _st),
    "nva_step_prepare_decode": ([_vp, _pseq, _ci, _ci], _st),
    "nva_norm_rope_attention_forward": ([_vp, _vp, _vp, _pnorm, _pnorm, _pnorm,
                                         ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _ci, _vp, _vp,
                                         _vp], _st),
    "nva_qkv_norm_rope_attention_forward": ([_vp, _vp, _vp, _pnorm, _pnorm, _pnorm,
                                             ctypes.POINTER(AttnDesc), _vp, _ci, _vp, _vp, _vp],
                                            _st),
}

_lib = None


def load():
    """Load libnva.so and declare its signatures; raises ImportError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; "
                "g.build()' or make -C nano-vllm-java_amd/csrc)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib
