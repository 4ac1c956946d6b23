"""ctypes binding of libpokit_hip.so (the C ABI declared in include/pokit_hip.h).

The library is loaded from this package directory.  There is no fallback: if
it is missing, importing the HIP backend raises, so nothing can silently run
on another path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpokit_hip.so")

STATUS_OK = 0
STATUS_INVALID_ARGUMENT = 1
STATUS_RUNTIME_ERROR = 2
STATUS_BUFFER_TOO_SMALL = 3
STATUS_INTERNAL_ERROR = 4
STATUS_UNSUPPORTED = 5
NO_EXPERT = 0xFFFFFFFF

# Every symbol include/pokit_hip.h declares.
EXPORTS = (
    "pk_hip_version", "pk_hip_type_supported", "pk_hip_create", "pk_hip_destroy",
    "pk_hip_upload", "pk_hip_upload_device", "pk_hip_weight_release", "pk_hip_weight_bytes",
    "pk_hip_weight_device_ptr", "pk_hip_matvec", "pk_hip_matvec_async", "pk_hip_moe_decode",
    "pk_hip_moe_decode_async", "pk_hip_moe35_decode", "pk_hip_moe35_decode_async", "pk_hip_sync",
    "pk_hip_get_stats", "pk_hip_reset_stats",
    "pk_hip_set_kernel_timing", "pk_hip_device_name", "pk_hip_moe_prefill",
    "pk_hip_moe35_prefill", "pk_hip_moe35_prefill_async",
    "pk_hip_moe_prefill_async", "pk_hip_qwen3moe_create", "pk_hip_qwen3moe_destroy",
    "pk_hip_qwen3moe_generate", "pk_hip_synth_weight", "pk_hip_matvec_reference_order",
    "pk_hip_weight_download", "pk_hip_moe_decode_noalloc", "pk_hip_dequantize_rows",
    "pk_hip_expf_block_sums", "pk_hip_rmsnorm", "pk_hip_add_rmsnorm", "pk_hip_matvec_add_rmsnorm", "pk_hip_attention_steps",
    "pk_hip_read_floor_async", "pk_hip_moe_decode_traced_async", "pk_hip_set_libm_expf",
    "pk_hip_moe_decode_reference_order",
)
TRACE_WORDS = 3 * 8192 * 8


class Options(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("time_kernels", ctypes.c_uint32)]


class Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "matvec_calls", "moe_decode_calls", "dispatches", "q4_0_dispatches", "q8_0_dispatches",
        "q4_k_dispatches", "q5_k_dispatches", "q6_k_dispatches", "float_dispatches",
        "weight_bytes", "resident_bytes", "uploaded_bytes", "router_fallbacks",
        "router_candidates", "expert_hits", "expert_misses", "matvec_ns", "router_ns",
        "gate_up_ns", "down_ns", "router_launches", "gate_up_launches", "down_launches",
        "matvec_launches", "prefill_calls", "prefill_tokens", "prefill_ns",
        "prefill_route_ns", "prefill_gate_up_ns", "prefill_down_ns", "q4_1_dispatches",
        "q5_0_dispatches", "q5_1_dispatches", "q2_k_dispatches", "q3_k_dispatches")]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class MoeLayerDesc(ctypes.Structure):
    _fields_ = [("router", ctypes.c_void_p), ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p),
                ("down", ctypes.c_void_p), ("top_k", ctypes.c_uint32),
                ("normalize", ctypes.c_uint32), ("scale", ctypes.c_float)]


class Moe35LayerDesc(ctypes.Structure):
    _fields_ = [("routed", MoeLayerDesc), ("shared_router", ctypes.c_void_p),
                ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p),
                ("shared_down", ctypes.c_void_p)]


class Qwen3MoeConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "layers", "hidden", "heads", "kv_heads", "head_dim", "experts", "top_k", "ffn", "vocab",
        "kv_capacity", "context", "normalize", "reference_order")] + [
        ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
        ("libm_expf_pairs", ctypes.c_void_p), ("libm_expf_count", ctypes.c_uint64)]


class Qwen3MoeLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "attn_norm", "q", "q_norm", "k", "k_norm", "v", "o", "ffn_norm", "router", "gate", "up",
        "down")]


class Qwen3MoeWeights(ctypes.Structure):
    _fields_ = [("token_embd", ctypes.c_void_p), ("output_norm", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("layers", ctypes.POINTER(Qwen3MoeLayer))]


class AttentionConfig(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("capacity", ctypes.c_uint32),
                ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
                ("reference_order", ctypes.c_uint32), ("libm_expf_pairs", ctypes.c_void_p),
                ("libm_expf_count", ctypes.c_uint64)]


class GenerationStats(ctypes.Structure):
    _fields_ = [("prefill_ns", ctypes.c_uint64), ("decode_ns", ctypes.c_uint64),
                ("prompt_tokens", ctypes.c_uint32), ("decode_forwards", ctypes.c_uint32)]


_lib = None


def lib() -> ctypes.CDLL:
    """Load libpokit_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m pokitlms_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    vp, u32, u64, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t
    cp = ctypes.c_char_p
    fp = ctypes.POINTER(ctypes.c_float)
    up = ctypes.POINTER(ctypes.c_uint32)
    L.pk_hip_version.restype = ctypes.c_char_p
    L.pk_hip_version.argtypes = []
    L.pk_hip_type_supported.restype = ctypes.c_int
    L.pk_hip_type_supported.argtypes = [u32]
    L.pk_hip_create.restype = ctypes.c_int
    L.pk_hip_create.argtypes = [ctypes.c_int, ctypes.POINTER(Options), ctypes.POINTER(vp), cp, sz]
    L.pk_hip_destroy.restype = None
    L.pk_hip_destroy.argtypes = [vp]
    for name in ("pk_hip_upload", "pk_hip_upload_device"):
        f = getattr(L, name)
        f.restype = ctypes.c_int
        f.argtypes = [vp, u32, u64, u64, u32, vp, u64, ctypes.POINTER(vp), cp, sz]
    L.pk_hip_weight_release.restype = None
    L.pk_hip_weight_release.argtypes = [vp]
    L.pk_hip_weight_bytes.restype = u64
    L.pk_hip_weight_bytes.argtypes = [vp]
    L.pk_hip_weight_device_ptr.restype = vp
    L.pk_hip_weight_device_ptr.argtypes = [vp]
    L.pk_hip_dequantize_rows.restype = ctypes.c_int
    L.pk_hip_dequantize_rows.argtypes = [vp, vp, ctypes.c_uint32, u64, ctypes.c_uint32, vp,
                                         ctypes.c_char_p, ctypes.c_size_t]
    L.pk_hip_expf_block_sums.restype = ctypes.c_int
    L.pk_hip_expf_block_sums.argtypes = [vp, vp, u64, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, vp, ctypes.c_char_p, ctypes.c_size_t]
    L.pk_hip_rmsnorm.restype = ctypes.c_int
    L.pk_hip_rmsnorm.argtypes = [vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float, vp,
                                 ctypes.c_char_p, ctypes.c_size_t]
    L.pk_hip_add_rmsnorm.restype = ctypes.c_int
    L.pk_hip_add_rmsnorm.argtypes = [vp, vp, vp, vp, u32, u32, ctypes.c_float, vp, vp, cp, sz]
    L.pk_hip_matvec_add_rmsnorm.restype = ctypes.c_int
    L.pk_hip_matvec_add_rmsnorm.argtypes = [vp, vp, vp, vp, vp, ctypes.c_float, vp, vp, cp, sz]
    L.pk_hip_attention_steps.restype = ctypes.c_int
    L.pk_hip_attention_steps.argtypes = [vp, ctypes.POINTER(AttentionConfig), vp, vp, u32, vp, vp,
                                         vp, vp, cp, sz]
    L.pk_hip_read_floor_async.restype = ctypes.c_int
    L.pk_hip_read_floor_async.argtypes = [vp, vp, u64, vp, vp, cp, sz]
    L.pk_hip_weight_download.restype = ctypes.c_int
    L.pk_hip_weight_download.argtypes = [vp, vp, u64, ctypes.c_char_p, ctypes.c_size_t]
    L.pk_hip_matvec.restype = ctypes.c_int
    L.pk_hip_matvec.argtypes = [vp, vp, u32, fp, u32, fp, cp, sz]
    L.pk_hip_matvec_reference_order.restype = ctypes.c_int
    L.pk_hip_matvec_reference_order.argtypes = [vp, vp, u32, fp, fp, cp, sz]
    L.pk_hip_matvec_async.restype = ctypes.c_int
    L.pk_hip_matvec_async.argtypes = [vp, vp, u32, vp, u32, vp, vp, cp, sz]
    L.pk_hip_moe_decode.restype = ctypes.c_int
    L.pk_hip_moe_decode.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), fp, fp, up, fp, cp, sz]
    L.pk_hip_moe35_decode.restype = ctypes.c_int
    L.pk_hip_moe35_decode.argtypes = [vp, ctypes.POINTER(Moe35LayerDesc), fp, fp, up, fp, cp, sz]
    L.pk_hip_moe35_decode_async.restype = ctypes.c_int
    L.pk_hip_moe35_decode_async.argtypes = [vp, ctypes.POINTER(Moe35LayerDesc), vp, vp, vp, vp,
                                            vp, cp, sz]
    L.pk_hip_moe_decode_async.restype = ctypes.c_int
    L.pk_hip_moe_decode_async.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), vp, vp, vp, vp, vp,
                                          cp, sz]
    L.pk_hip_set_libm_expf.restype = ctypes.c_int
    L.pk_hip_set_libm_expf.argtypes = [vp, vp, u64, cp, sz]
    L.pk_hip_moe_decode_reference_order.restype = ctypes.c_int
    L.pk_hip_moe_decode_reference_order.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), fp, fp, up,
                                                    fp, cp, sz]
    L.pk_hip_moe_decode_traced_async.restype = ctypes.c_int
    L.pk_hip_moe_decode_traced_async.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), vp, vp, vp, vp,
                                                 vp, vp, cp, sz]
    L.pk_hip_moe_decode_noalloc.restype = ctypes.c_int
    L.pk_hip_moe_decode_noalloc.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), vp, vp, vp, vp, vp,
                                            cp, sz]
    L.pk_hip_sync.restype = ctypes.c_int
    L.pk_hip_sync.argtypes = [vp, vp, cp, sz]
    L.pk_hip_get_stats.restype = ctypes.c_int
    L.pk_hip_get_stats.argtypes = [vp, ctypes.POINTER(Stats)]
    L.pk_hip_reset_stats.restype = None
    L.pk_hip_reset_stats.argtypes = [vp]
    L.pk_hip_set_kernel_timing.restype = ctypes.c_int
    L.pk_hip_set_kernel_timing.argtypes = [vp, ctypes.c_int]
    L.pk_hip_device_name.restype = ctypes.c_int
    L.pk_hip_moe_prefill.restype = ctypes.c_int
    L.pk_hip_moe_prefill.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), fp, u32, fp, up, fp, cp, sz]
    L.pk_hip_moe_prefill_async.restype = ctypes.c_int
    L.pk_hip_moe_prefill_async.argtypes = [vp, ctypes.POINTER(MoeLayerDesc), vp, u32, vp, vp, vp,
                                           vp, cp, sz]
    L.pk_hip_moe35_prefill.restype = ctypes.c_int
    L.pk_hip_moe35_prefill.argtypes = [vp, ctypes.POINTER(Moe35LayerDesc), fp, u32, fp, up, fp,
                                       cp, sz]
    L.pk_hip_moe35_prefill_async.restype = ctypes.c_int
    L.pk_hip_moe35_prefill_async.argtypes = [vp, ctypes.POINTER(Moe35LayerDesc), vp, u32, vp, vp,
                                             vp, vp, cp, sz]
    L.pk_hip_device_name.argtypes = [vp, cp, sz]
    L.pk_hip_qwen3moe_create.restype = ctypes.c_int
    L.pk_hip_qwen3moe_create.argtypes = [vp, ctypes.POINTER(Qwen3MoeConfig),
                                         ctypes.POINTER(Qwen3MoeWeights), ctypes.POINTER(vp), cp, sz]
    L.pk_hip_qwen3moe_destroy.restype = None
    L.pk_hip_qwen3moe_destroy.argtypes = [vp]
    L.pk_hip_qwen3moe_generate.restype = ctypes.c_int
    L.pk_hip_qwen3moe_generate.argtypes = [vp, up, u32, u32, up, fp,
                                           ctypes.POINTER(GenerationStats), cp, sz]
    L.pk_hip_synth_weight.restype = ctypes.c_int
    L.pk_hip_synth_weight.argtypes = [vp, u32, u64, u64, u32, u64, u32, ctypes.POINTER(vp), cp, sz]
    _lib = L
    return L
