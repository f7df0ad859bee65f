"""ctypes bindings of the MI355X RINA decode-path libraries.

The product is native: lib/librina_hip.so (gfx950 kernels behind the C-ABI
of include/rina_hip.h) and lib/librina_engine.so (the C++ Inference engine,
include/rina_engine.h).  This module only loads them and declares their
signatures for Python callers (tests, bench).  There is no Python or CPU
fallback: a missing library raises.
"""
import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")

# quant types (core/quant.h) and KV modes / formats (include/rina_hip.h)
QT_Q4_0, QT_FP32, QT_Q4_0F, QT_Q2_K = 5, 6, 7, 10
KV_MODES = {"fp32": 0, "q8": 1, "q4": 2, "q4k_q2v": 3, "q2": 4, "q2k_q1v": 5}
KVF_Q8_0, KVF_Q4_0, KVF_Q2_1, KVF_Q1_0 = 1, 2, 3, 4
EPI_STORE, EPI_ADD, EPI_SWIGLU = 0, 1, 2
PRO_NONE, PRO_RMSNORM, PRO_LAYERNORM = 0, 1, 2
STATUS = {0: "OK", -1: "ERR_ARG", -2: "ERR_QTYPE", -3: "ERR_SHAPE", -4: "ERR_RANGE", -5: "ERR_HIP",
          -6: "ERR_WORKSPACE"}

_hip = None
_eng = None

VP, I32, I64, F32, SZ = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t


class LinearSeg(C.Structure):
    _fields_ = [("weight", VP), ("weight2", VP), ("out", VP), ("N", I32)]


_HIP_SIGS = {
    "rina_hip_linear": (I32, [VP, I32, VP, VP, I32, I32, I32, VP]),
    "rina_hip_linear_fused": (I32, [C.POINTER(LinearSeg), I32, I32, VP, I32, I32, I32, I32, VP, F32, VP]),
    "rina_hip_linear_fused_ex": (I32, [C.POINTER(LinearSeg), I32, I32, VP, I32, I32, I32, I32, VP, F32, VP, VP]),
    "rina_hip_pack_weights": (I32, [I32, VP, I64, VP, VP]),
    "rina_hip_dequant_weights": (I32, [I32, VP, I64, VP, VP]),
    "rina_hip_pack_weights_hf": (I32, [VP, I64, VP, VP]),
    "rina_hip_kv_quantize": (I32, [I32, VP, VP, I64, VP]),
    "rina_hip_kv_dequant": (I32, [I32, VP, VP, I64, VP]),
    "rina_hip_kv_region_bytes": (SZ, [I32, I32, I32, I32]),
    "rina_hip_rope_append": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, I32, I32, I32, I32, I32, I32, VP, I32,
                                   VP]),
    "rina_hip_gqa_attention_workspace": (SZ, [I32, I32, I32, I32]),
    "rina_hip_gqa_attention": (I32, [VP, VP, VP, VP, VP, I32, I32, VP, VP, I32, I32, I32, I32, I32, VP, I32, VP,
                                     VP, SZ, VP]),
    "rina_hip_gqa_decode_attention": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, I32, I32, I32, I32, VP, I32,
                                            VP, VP, VP, SZ, VP]),
    "rina_hip_noalloc_scratch_bytes": (SZ, []),
    "rina_hip_gqa_decode_attention_noalloc": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, I32, I32, I32, I32, VP,
                                                    I32, VP, VP, VP]),
    "rina_hip_mla_attention_workspace": (SZ, [I32, I32, I32, I32]),
    "rina_hip_mla_cache_bytes": (SZ, [I32, I32, I32]),
    "rina_hip_mla_decode_attention": (I32, [VP, VP, VP, F32, VP, VP, VP, I32, VP, I32, I32, I32, I32, I32, I32, VP,
                                            I32, VP, VP, SZ, VP]),
    "rina_hip_mla_fused_positions": (I32, []),
    "rina_hip_gqa_one_launch_positions": (I32, []),
    "rina_hip_mla_decode_attention_ex": (I32, [VP, VP, VP, F32, VP, VP, VP, I32, VP, I32, I32, I32, I32, I32, I32,
                                               VP, I32, I32, VP, VP, SZ, VP]),
    "rina_hip_mla_prompt_workspace": (SZ, [I32, I32, I32, I32, I32, I32]),
    "rina_hip_mla_prompt_attention": (I32, [VP, VP, VP, F32, VP, VP, VP, I32, VP, I32, I32, I32, I32, I32, I32, I32,
                                            VP, VP, SZ, VP]),
    "rina_hip_moe_topk": (I32, [VP, I32, I32, VP, VP, VP]),
    "rina_hip_moe_workspace": (SZ, [I32, I32]),
    "rina_hip_moe_rows_workspace": (SZ, [I32, I32, I32, I32, I32, I32]),
    "rina_hip_moe_rows": (I32, [VP, I32, VP, F32, VP, I32, VP, VP, VP, I32, I32, VP, VP, VP, I32, I64, I64, I32, I32,
                                I32, I32, VP, SZ, VP]),
    "rina_hip_moe_ffn": (I32, [VP, VP, VP, VP, I32, I64, I64, I32, VP, VP, I32, I32, I32, VP, VP, VP, SZ, VP]),
    "rina_hip_moe_block_workspace": (SZ, [I32, I32, I32, I32, I32]),
    "rina_hip_moe_block": (I32, [VP, VP, F32, VP, I32, VP, VP, VP, I32, VP, VP, VP, I32, I64, I64, I32, I32, I32,
                                 I32, VP, SZ, VP]),
    "rina_hip_ssm_step": (I32, [VP, VP, I32, I32, I32, VP, VP, VP, I32, VP]),
    "rina_hip_ssm_scan": (I32, [VP, VP, I32, I32, I32, I32, VP, VP, VP, I32, I32, VP]),
    "rina_hip_ssm_proj_step": (I32, [VP, VP, F32, C.POINTER(VP), C.POINTER(VP), I32, I32, I32, I32, I32, VP, VP,
                                     VP, I32, VP]),
    "rina_hip_dq_attention_workspace": (SZ, [I32, I32, I32]),
    "rina_hip_dq_decode_attention": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, I32, I32, I32, I32, I32, VP,
                                           I32, VP, VP, SZ, VP]),
    "rina_hip_dq_prompt_workspace": (SZ, [I32, I32, I32, I32, I32, I32]),
    "rina_hip_dq_prompt_attention": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, I32, I32, I32, I32, I32, I32,
                                           VP, VP, SZ, VP]),
    "rina_hip_dq_kv_region_bytes": (SZ, [I32, I32, I32, I32, I32, I32, I32]),
    "rina_hip_dq_decode_attention_kv": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, VP, VP, VP, I32, I32, I32, I32,
                                              I32, I32, VP, I32, VP, VP, SZ, VP]),
    "rina_hip_dq_prompt_attention_kv": (I32, [VP, VP, VP, VP, VP, VP, VP, VP, VP, I32, VP, VP, VP, I32, I32, I32, I32,
                                              I32, I32, I32, I32, VP, VP]),
    "rina_hip_rms_norm": (I32, [VP, VP, VP, I32, I32, F32, VP]),
    "rina_hip_layer_norm": (I32, [VP, VP, VP, I32, I32, F32, VP]),
    "rina_hip_rope": (I32, [VP, VP, VP, I32, I32, I32, I32, VP, I32, VP]),
    "rina_hip_embedding": (I32, [VP, I32, VP, VP, VP, I32, I32, I32, VP]),
    "rina_hip_silu_mul": (I32, [VP, VP, VP, I64, VP]),
    "rina_hip_add": (I32, [VP, VP, VP, I64, VP]),
    "rina_hip_saxpy": (I32, [VP, VP, F32, I64, VP]),
    "rina_hip_argmax": (I32, [VP, I32, VP, VP, VP, VP]),
    "rina_hip_argmax_ws": (I32, [VP, I32, VP, VP, VP, VP, VP]),
    "rina_hip_read_probe": (I32, [VP, I64, I32, VP, VP]),
    "rina_hip_linear_argmax": (I32, [VP, I32, VP, I32, I32, VP, F32, VP, I32, VP, VP]),
    "rina_hip_argmax_partial": (I32, [VP, I32, VP, VP]),
    "rina_hip_argmax_embed": (I32, [VP, I32, I32, VP, VP, VP, VP, I32, VP, I32, I32, VP]),
    "rina_hip_version": (C.c_char_p, []),
}

_ENG_SIGS = {
    "rina_model_create": (VP, [C.c_char_p]),
    "rina_model_destroy": (None, [VP]),
    "rina_model_load": (VP, [C.c_char_p]),
    "rina_model_add_tensor": (I32, [VP, C.c_char_p, I32, I32, C.POINTER(I64), VP]),
    "rina_infer_create": (VP, [VP, C.c_char_p, C.c_char_p, I32]),
    "rina_infer_destroy": (None, [VP]),
    "rina_infer_forward": (I32, [VP, VP, VP, I32, I32, I32, VP]),
    "rina_infer_generate": (I32, [VP, C.POINTER(I32), I32, I32, C.POINTER(I32), I32, VP, C.POINTER(F32)]),
    "rina_infer_decode": (I32, [VP, I32, C.POINTER(I32), I32, VP, C.POINTER(F32)]),
    "rina_infer_kv_region": (I32, [VP, I32, I32, C.POINTER(VP), C.POINTER(SZ)]),
    "rina_infer_set_kv_tap": (I32, [VP, VP]),
    "rina_engine_last_error": (C.c_char_p, []),
}


def _declare(lib, sigs):
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def hip_path():
    return os.path.join(LIB_DIR, "librina_hip.so")


def engine_path():
    # RINA_ENGINE_SO: the sanitizer build of the same host sources (tests)
    return os.environ.get("RINA_ENGINE_SO") or os.path.join(LIB_DIR, "librina_engine.so")


def load_hip():
    """Load librina_hip.so (raises if it has not been built)."""
    global _hip
    if _hip is None:
        p = hip_path()
        if not os.path.exists(p):
            raise RuntimeError("librina_hip.so not built (run __graft_entry__.build()): %s" % p)
        _hip = _declare(C.CDLL(p, mode=C.RTLD_GLOBAL), _HIP_SIGS)
    return _hip


def load_engine():
    """Load librina_engine.so (and librina_hip.so first)."""
    global _eng
    if _eng is None:
        load_hip()
        p = engine_path()
        if not os.path.exists(p):
            raise RuntimeError("librina_engine.so not built (run __graft_entry__.build()): %s" % p)
        _eng = _declare(C.CDLL(p, mode=C.RTLD_GLOBAL), _ENG_SIGS)
    return _eng


def check(rc, what=""):
    if rc != 0:
        msg = STATUS.get(rc, str(rc))
        extra = ""
        if _eng is not None:
            e = _eng.rina_engine_last_error()
            extra = (" (%s)" % e.decode()) if e else ""
        raise RuntimeError("%s failed: %s%s" % (what, msg, extra))
    return rc
