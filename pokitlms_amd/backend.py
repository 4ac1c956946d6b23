"""Python host API over libpokit_hip.so.

Mirrors the reference plugin surface for the routed-MoE path:

* ``HipBackend.try_linear(tensor, x, y) -> bool`` is
  ``TensorLinearBackend::try_linear`` (include/pokitlms/model/tensor_linear.hpp:
  11-18 of the reference): False means "not covered, use the CPU kernel";
  shape errors raise ``ValueError``; device failures raise ``HipError`` and
  leave the backend failed (src/vulkan_linear.cpp:636, 731-735).
* ``HipBackend.upload(..., n_experts=E)`` keeps every expert resident in HBM,
  replacing ExpertStore's LRU (src/expert_store.cpp:81-141).
* ``HipBackend.moe_decode(layer, x)`` is the MoE block of
  src/qwen3_moe_runner.cpp:643-692 for one token.

Everything here is plumbing around the C ABI; the arithmetic runs in the HIP
kernels of ``csrc/``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _abi
from . import synth as S

_ERRBUF = 512


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


class Unsupported(HipError):
    pass


def _raise(status: int, err: ctypes.Array) -> None:
    if status == _abi.STATUS_OK:
        return
    msg = err.value.decode(errors="replace")
    if status == _abi.STATUS_UNSUPPORTED:
        raise Unsupported(status, msg)
    if status == _abi.STATUS_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise HipError(status, msg)


def _f32p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


@dataclass
class TensorView:
    """A GGUF tensor as the reference's TensorReader presents it: type,
    dims = [in, out], and the encoded payload (host bytes)."""
    gtype: int
    dims: tuple
    payload: np.ndarray


class Weight:
    def __init__(self, backend: "HipBackend", handle: int, gtype: int, in_features: int,
                 out_features: int, n_experts: int, nbytes: int):
        self.backend, self.handle = backend, handle
        self.gtype, self.in_features, self.out_features = gtype, in_features, out_features
        self.n_experts, self.nbytes = n_experts, nbytes

    @property
    def device_ptr(self) -> int:
        return _abi.lib().pk_hip_weight_device_ptr(self.handle) or 0

    @property
    def slice_bytes(self) -> int:
        return self.nbytes // max(self.n_experts, 1)

    def download(self) -> np.ndarray:
        """The weight's GGUF encoding, read back from HBM (uint8[nbytes])."""
        out = np.empty(self.nbytes, dtype=np.uint8)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_weight_download(self.handle, out.ctypes.data, self.nbytes, err,
                                                 _ERRBUF), err)
        return out

    def release(self) -> None:
        if self.handle:
            _abi.lib().pk_hip_weight_release(self.handle)
            self.handle = None


class MoeLayerHandles:
    """A routed MoE layer resident in HBM (router, gate, up, down)."""

    def __init__(self, router: Weight, gate: Weight, up: Weight, down: Weight, top_k: int,
                 normalize: bool, scale: float = 1.0):
        self.router, self.gate, self.up, self.down = router, gate, up, down
        self.top_k, self.normalize, self.scale = top_k, normalize, scale
        self.desc = _abi.MoeLayerDesc(router.handle, gate.handle, up.handle, down.handle, top_k,
                                      1 if normalize else 0, scale)
        self.hidden, self.ffn, self.experts = router.in_features, gate.out_features, router.out_features

    def routed_bytes(self) -> int:
        return self.router.nbytes + self.top_k * (self.gate.slice_bytes + self.up.slice_bytes +
                                                  self.down.slice_bytes)

    def release(self) -> None:
        for w in (self.router, self.gate, self.up, self.down):
            w.release()


class Moe35LayerHandles(MoeLayerHandles):
    """A Qwen3.5-MoE layer resident in HBM: the routed experts plus the shared
    expert (router vector, gate, up, down); ``scale`` = expert_weights_scale."""

    def __init__(self, routed: MoeLayerHandles, shared_router: Weight, shared_gate: Weight,
                 shared_up: Weight, shared_down: Weight):
        super().__init__(routed.router, routed.gate, routed.up, routed.down, routed.top_k,
                         routed.normalize, routed.scale)
        self.shared = (shared_router, shared_gate, shared_up, shared_down)
        self.desc35 = _abi.Moe35LayerDesc(self.desc, shared_router.handle, shared_gate.handle,
                                          shared_up.handle, shared_down.handle)

    def routed_bytes(self) -> int:
        return super().routed_bytes() + sum(w.nbytes for w in self.shared)

    def release(self) -> None:
        super().release()
        for w in self.shared:
            w.release()


class HipBackend:
    def __init__(self, device: int = 0, time_kernels: bool = False):
        L = _abi.lib()
        opts = _abi.Options(ctypes.sizeof(_abi.Options), 1 if time_kernels else 0)
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(L.pk_hip_create(device, ctypes.byref(opts), ctypes.byref(h), err, _ERRBUF), err)
        self.handle = h.value
        self._cache = {}

    # ---- lifetime ---------------------------------------------------------------
    def close(self) -> None:
        for w in self._cache.values():
            w.release()
        self._cache.clear()
        if self.handle:
            _abi.lib().pk_hip_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- weights ----------------------------------------------------------------
    def upload(self, gtype: int, in_features: int, out_features: int, data: np.ndarray,
               n_experts: int = 0) -> Weight:
        buf = np.ascontiguousarray(data).view(np.uint8)
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_upload(self.handle, gtype, in_features, out_features, n_experts,
                                        buf.ctypes.data, buf.nbytes, ctypes.byref(h), err,
                                        _ERRBUF), err)
        return Weight(self, h.value, gtype, in_features, out_features, n_experts, buf.nbytes)

    def upload_device(self, gtype: int, in_features: int, out_features: int, device_ptr: int,
                      nbytes: int, n_experts: int = 0) -> Weight:
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_upload_device(self.handle, gtype, in_features, out_features,
                                               n_experts, device_ptr, nbytes, ctypes.byref(h),
                                               err, _ERRBUF), err)
        return Weight(self, h.value, gtype, in_features, out_features, n_experts, nbytes)

    def upload_moe_layer(self, layer: "S.MoeLayer") -> MoeLayerHandles:
        r = self.upload(S.F32, layer.hidden, layer.experts, layer.router)
        g = self.upload(layer.gate_type, layer.hidden, layer.ffn, layer.gate, layer.experts)
        u = self.upload(layer.up_type, layer.hidden, layer.ffn, layer.up, layer.experts)
        d = self.upload(layer.down_type, layer.ffn, layer.hidden, layer.down, layer.experts)
        return MoeLayerHandles(r, g, u, d, layer.top_k, layer.normalize)

    def upload_moe35_layer(self, layer: "S.Moe35Layer") -> Moe35LayerHandles:
        routed = self.upload_moe_layer(layer)
        routed = MoeLayerHandles(routed.router, routed.gate, routed.up, routed.down, layer.top_k,
                                 layer.normalize, layer.scale)
        sr = self.upload(S.F32, layer.hidden, 1, layer.shared_router)
        sg = self.upload(layer.gate_type, layer.hidden, layer.shared_ffn, layer.shared_gate)
        su = self.upload(layer.up_type, layer.hidden, layer.shared_ffn, layer.shared_up)
        sd = self.upload(layer.down_type, layer.shared_ffn, layer.hidden, layer.shared_down)
        return Moe35LayerHandles(routed, sr, sg, su, sd)

    # ---- matvec -----------------------------------------------------------------
    def matvec(self, w: Weight, x: np.ndarray, expert: int | None = None) -> np.ndarray:
        xx = np.ascontiguousarray(x, dtype=np.float32)
        batch = 1 if xx.ndim == 1 else xx.shape[0]
        if xx.size != batch * w.in_features:
            raise ValueError("input width does not match the matrix")
        y = np.empty((batch, w.out_features), dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_matvec(self.handle, w.handle,
                                        _abi.NO_EXPERT if expert is None else expert, _f32p(xx),
                                        batch, _f32p(y), err, _ERRBUF), err)
        return y[0] if xx.ndim == 1 else y

    def matvec_reference_order(self, w: Weight, x: np.ndarray,
                               expert: int | None = None) -> np.ndarray:
        """W . x summed in the CPU's order (bit-equal to the reference)."""
        xx = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        y = np.empty(w.out_features, dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_matvec_reference_order(
            self.handle, w.handle, _abi.NO_EXPERT if expert is None else expert, _f32p(xx),
            _f32p(y), err, _ERRBUF), err)
        return y

    def matvec_async(self, w: Weight, device_x: int, batch: int, device_y: int, stream: int = 0,
                     expert: int | None = None) -> None:
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_matvec_async(self.handle, w.handle,
                                              _abi.NO_EXPERT if expert is None else expert,
                                              device_x, batch, device_y, stream or None, err,
                                              _ERRBUF), err)

    def try_linear(self, tensor: TensorView, x: np.ndarray, y: np.ndarray) -> bool:
        """TensorLinearBackend::try_linear over a host GGUF tensor (uploaded
        once per payload object and kept resident)."""
        if not _abi.lib().pk_hip_type_supported(tensor.gtype):
            return False
        in_features, out_features = int(tensor.dims[0]), int(tensor.dims[1])
        if x.size != in_features or y.size != out_features:
            raise ValueError("GGUF matrix dimensions do not match linear input/output")
        key = id(tensor.payload)
        w = self._cache.get(key)
        if w is None or w.gtype != tensor.gtype:
            try:
                w = self.upload(tensor.gtype, in_features, out_features, tensor.payload)
            except Unsupported:
                return False
            self._cache[key] = w
        try:
            y[...] = self.matvec(w, x)
        except Unsupported:
            return False
        return True

    # ---- MoE --------------------------------------------------------------------
    def moe_decode(self, layer: MoeLayerHandles, x: np.ndarray):
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(layer.hidden, dtype=np.float32)
        ids = np.zeros(layer.top_k, dtype=np.uint32)
        probs = np.zeros(layer.top_k, dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_decode(self.handle, ctypes.byref(layer.desc), _f32p(xx),
                                            _f32p(y), ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                            _f32p(probs), err, _ERRBUF), err)
        return y, ids, probs

    def moe35_decode(self, layer: Moe35LayerHandles, x: np.ndarray):
        """The Qwen3.5-MoE block (src/qwen35_runner.cpp:670-764): mixer output,
        route ids and weights (times expert_weights_scale)."""
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(layer.hidden, dtype=np.float32)
        ids = np.zeros(layer.top_k, dtype=np.uint32)
        w = np.zeros(layer.top_k, dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe35_decode(self.handle, ctypes.byref(layer.desc35), _f32p(xx),
                                              _f32p(y),
                                              ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                              _f32p(w), err, _ERRBUF), err)
        return y, ids, w

    def moe35_decode_async(self, layer: Moe35LayerHandles, device_x: int, device_y: int,
                           device_ids: int, device_weights: int, stream: int = 0) -> None:
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe35_decode_async(self.handle, ctypes.byref(layer.desc35),
                                                    device_x, device_y, device_ids,
                                                    device_weights, stream or None, err,
                                                    _ERRBUF), err)

    def moe35_prefill(self, layer: Moe35LayerHandles, x: np.ndarray):
        """A batch of tokens x [tokens, hidden] through the Qwen3.5-MoE block;
        per token the result of moe35_decode."""
        xx = np.ascontiguousarray(x, dtype=np.float32)
        if xx.ndim != 2 or xx.shape[1] != layer.hidden:
            raise ValueError(f"x must be [tokens, {layer.hidden}], got {xx.shape}")
        tokens = xx.shape[0]
        y = np.empty((tokens, layer.hidden), dtype=np.float32)
        ids = np.zeros((tokens, layer.top_k), dtype=np.uint32)
        w = np.zeros((tokens, layer.top_k), dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe35_prefill(self.handle, ctypes.byref(layer.desc35), _f32p(xx),
                                               tokens, _f32p(y),
                                               ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                               _f32p(w), err, _ERRBUF), err)
        return y, ids, w

    def moe35_prefill_async(self, layer: Moe35LayerHandles, device_x: int, tokens: int,
                            device_y: int, device_ids: int, device_weights: int,
                            stream: int = 0) -> None:
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe35_prefill_async(self.handle, ctypes.byref(layer.desc35),
                                                     device_x, tokens, device_y, device_ids,
                                                     device_weights, stream or None, err,
                                                     _ERRBUF), err)

    def moe_decode_async(self, layer: MoeLayerHandles, device_x: int, device_y: int,
                         device_ids: int, device_probs: int, stream: int = 0) -> None:
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_decode_async(self.handle, ctypes.byref(layer.desc),
                                                  device_x, device_y, device_ids, device_probs,
                                                  stream or None, err, _ERRBUF), err)

    def set_libm_expf(self, pairs) -> None:
        """The host libm's expf exceptions (uint32 [n, 2]) for the reference-order
        kernels of this context; None or empty clears them."""
        p = np.ascontiguousarray(pairs if pairs is not None else np.zeros((0, 2)), dtype=np.uint32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_set_libm_expf(self.handle, p.ctypes.data if p.size else None,
                                               p.size // 2, err, _ERRBUF), err)

    def moe_decode_reference_order(self, layer: MoeLayerHandles, x: np.ndarray):
        """The MoE block in the reference's operation order: (moe_result,
        ids, probs), bit for bit the reference's with the libm expf table set."""
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(layer.hidden, np.float32)
        ids = np.empty(layer.top_k, np.uint32)
        probs = np.empty(layer.top_k, np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_decode_reference_order(
            self.handle, ctypes.byref(layer.desc), _f32p(xx), _f32p(y),
            ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), _f32p(probs), err, _ERRBUF), err)
        return y, ids, probs

    def moe_decode_traced_async(self, layer: MoeLayerHandles, device_x: int, device_y: int,
                                device_ids: int, device_probs: int, device_trace: int,
                                stream: int = 0) -> None:
        """moe_decode_async that records its phase times into device_trace
        (_abi.TRACE_WORDS uint64 words; layout in include/pokit_hip.h)."""
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_decode_traced_async(self.handle, ctypes.byref(layer.desc),
                                                         device_x, device_y, device_ids,
                                                         device_probs, device_trace,
                                                         stream or None, err, _ERRBUF), err)

    def dequantize_rows(self, w: Weight, first_row: int = 0, rows: int | None = None,
                        expert: int | None = None) -> np.ndarray:
        """Rows of a resident weight as FP32 (the reference's
        read_float_rows_into / dequantize_quantized_row)."""
        rows = w.out_features - first_row if rows is None else rows
        out = np.empty((rows, w.in_features), dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_dequantize_rows(self.handle, w.handle,
                                                 _abi.NO_EXPERT if expert is None else expert,
                                                 first_row, rows, out.ctypes.data, err, _ERRBUF),
               err)
        return out

    def rmsnorm(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        """rms_norm of each row of x (the reference's src/rms_norm.cpp:9-27),
        bit for bit."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, n = (1, x.size) if x.ndim == 1 else x.shape
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        if w.size != n:
            raise ValueError("weight size must equal the row width")
        out = np.empty_like(x)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_rmsnorm(self.handle, x.ctypes.data, w.ctypes.data, rows, n,
                                         float(eps), out.ctypes.data, err, _ERRBUF), err)
        return out

    def add_rmsnorm(self, hidden: np.ndarray, delta, w: np.ndarray, eps: float):
        """The fast decode's residual add + RMSNorm kernel on each row:
        (hidden + delta, rms_norm(hidden + delta, w)); delta may be None."""
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        rows, n = (1, h.size) if h.ndim == 1 else h.shape
        d = None if delta is None else np.ascontiguousarray(delta, dtype=np.float32)
        if d is not None and d.size != h.size:
            raise ValueError("delta must have the hidden rows' shape")
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        if w.size != n:
            raise ValueError("weight size must equal the row width")
        h_out, out = np.empty_like(h), np.empty_like(h)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_add_rmsnorm(self.handle, h.ctypes.data,
                                             None if d is None else d.ctypes.data, w.ctypes.data,
                                             rows, n, float(eps), h_out.ctypes.data,
                                             out.ctypes.data, err, _ERRBUF), err)
        return h_out, out

    def matvec_add_rmsnorm(self, w: Weight, hidden: np.ndarray, delta, norm_w: np.ndarray,
                           eps: float):
        """The fast decode's projection with the norm in its staging:
        (hidden + delta, W . rms_norm(hidden + delta, norm_w)); delta may be None."""
        h = np.ascontiguousarray(hidden, dtype=np.float32).reshape(-1)
        d = None if delta is None else np.ascontiguousarray(delta, dtype=np.float32).reshape(-1)
        nw = np.ascontiguousarray(norm_w, dtype=np.float32).reshape(-1)
        if h.size != w.in_features or nw.size != h.size or (d is not None and d.size != h.size):
            raise ValueError("hidden, delta and norm weight must have the matrix's width")
        h_out = np.empty_like(h)
        y = np.empty(w.out_features, dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_matvec_add_rmsnorm(self.handle, w.handle, h.ctypes.data,
                                                    None if d is None else d.ctypes.data,
                                                    nw.ctypes.data, float(eps), h_out.ctypes.data,
                                                    y.ctypes.data, err, _ERRBUF), err)
        return h_out, y

    def attention_steps(self, heads: int, kv_heads: int, head_dim: int, capacity: int,
                        eps: float, theta: float, q_norm, k_norm, q, k, v,
                        reference_order: bool = False, libm_expf_pairs=None) -> np.ndarray:
        """The decode's attention stage of one layer for positions 0 .. steps-1
        (pk_hip_attention_steps): out [steps][heads * head_dim]."""
        qq = np.ascontiguousarray(q, dtype=np.float32)
        kk = np.ascontiguousarray(k, dtype=np.float32)
        vv = np.ascontiguousarray(v, dtype=np.float32)
        steps = qq.shape[0]
        if qq.shape != (steps, heads * head_dim) or kk.shape != (steps, kv_heads * head_dim) \
                or vv.shape != kk.shape:
            raise ValueError("q [steps][heads*head_dim], k and v [steps][kv_heads*head_dim]")
        qn = np.ascontiguousarray(q_norm, dtype=np.float32)
        kn = np.ascontiguousarray(k_norm, dtype=np.float32)
        cfg = _abi.AttentionConfig(heads, kv_heads, head_dim, capacity, eps, theta,
                                   1 if reference_order else 0)
        pairs = None
        if reference_order and libm_expf_pairs is not None:
            pairs = np.ascontiguousarray(libm_expf_pairs, dtype=np.uint32)
            cfg.libm_expf_pairs = pairs.ctypes.data
            cfg.libm_expf_count = pairs.shape[0]
        out = np.empty((steps, heads * head_dim), np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_attention_steps(self.handle, ctypes.byref(cfg), qn.ctypes.data,
                                                 kn.ctypes.data, steps, qq.ctypes.data,
                                                 kk.ctypes.data, vv.ctypes.data, out.ctypes.data,
                                                 err, _ERRBUF), err)
        return out

    def read_floor_async(self, src_ptr: int, nbytes: int, sink_ptr: int, stream) -> None:
        """A plain streaming read of nbytes device bytes (the HBM floor)."""
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_read_floor_async(self.handle, src_ptr, nbytes, sink_ptr, stream,
                                                  err, _ERRBUF), err)

    def expf_block_sums(self, pairs: np.ndarray, first_bits: int, block_size: int,
                        n_blocks: int) -> np.ndarray:
        """Checksums of the reference-order expf over float bit patterns
        (see pk_hip_expf_block_sums)."""
        p = np.ascontiguousarray(pairs, dtype=np.uint32).reshape(-1)
        out = np.empty(n_blocks, dtype=np.uint64)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_expf_block_sums(self.handle, p.ctypes.data if p.size else None,
                                                 p.size // 2, first_bits, block_size, n_blocks,
                                                 out.ctypes.data, err, _ERRBUF), err)
        return out

    def moe_decode_noalloc(self, layer: MoeLayerHandles, device_x: int, device_y: int,
                           device_ids: int, device_probs: int, stream: int = 0) -> None:
        """moe_decode_async on the library's static device scratch (no device
        allocation; calls that overlap on one GPU race)."""
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_decode_noalloc(self.handle, ctypes.byref(layer.desc),
                                                    device_x, device_y, device_ids, device_probs,
                                                    stream or None, err, _ERRBUF), err)

    def moe_prefill(self, layer: MoeLayerHandles, x: np.ndarray):
        """A batch of tokens x [tokens, hidden] through the layer; per token the
        result of moe_decode (the reference's prompt loop, one token at a time:
        src/qwen3_moe_runner.cpp:785-790)."""
        xx = np.ascontiguousarray(x, dtype=np.float32)
        if xx.ndim != 2 or xx.shape[1] != layer.hidden:
            raise ValueError(f"x must be [tokens, {layer.hidden}], got {xx.shape}")
        tokens = xx.shape[0]
        y = np.empty((tokens, layer.hidden), dtype=np.float32)
        ids = np.zeros((tokens, layer.top_k), dtype=np.uint32)
        probs = np.zeros((tokens, layer.top_k), dtype=np.float32)
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_prefill(self.handle, ctypes.byref(layer.desc), _f32p(xx),
                                             tokens, _f32p(y),
                                             ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                             _f32p(probs), err, _ERRBUF), err)
        return y, ids, probs

    def moe_prefill_async(self, layer: MoeLayerHandles, device_x: int, tokens: int, device_y: int,
                          device_ids: int, device_probs: int, stream: int = 0) -> None:
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_moe_prefill_async(self.handle, ctypes.byref(layer.desc),
                                                   device_x, tokens, device_y, device_ids,
                                                   device_probs, stream or None, err, _ERRBUF),
               err)

    def sync(self, stream: int = 0) -> None:
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_sync(self.handle, stream or None, err, _ERRBUF), err)

    def stats(self) -> dict:
        st = _abi.Stats()
        _abi.lib().pk_hip_get_stats(self.handle, ctypes.byref(st))
        return st.as_dict()

    def reset_stats(self) -> None:
        _abi.lib().pk_hip_reset_stats(self.handle)

    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        st = _abi.lib().pk_hip_device_name(self.handle, buf, len(buf))
        if st not in (0, 3):
            _raise(st, buf)
        return buf.value.decode(errors="replace")

    def set_kernel_timing(self, enabled: bool) -> None:
        _abi.lib().pk_hip_set_kernel_timing(self.handle, 1 if enabled else 0)
