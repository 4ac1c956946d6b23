"""ctypes bindings to the parity oracle -- TEST INFRASTRUCTURE ONLY.

Two interchangeable back ends with one API:

* ``Oracle("port")``      -- oracle/libpk_oracle.so, the C restatement of the
  reference CPU path (oracle/pk_oracle.c).
* ``Oracle("reference")`` -- oracle/_ref/libpkref.so, the reference's own CPU
  sources compiled in place by ``make -C oracle ref`` (present only where the
  reference checkout was available at build time, or carried as a built file).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module; the product package never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_PATH = os.path.join(HERE, "libpk_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libpkref.so")
REFERENCE_ROOT = "/root/reference"

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u8p = ctypes.c_void_p


def build(reference: bool = True) -> None:
    """Compile the C restatement, and the reference library when its sources exist."""
    targets = ["all"]
    if reference and os.path.isdir(os.path.join(REFERENCE_ROOT, "src")):
        targets.append("ref")
        # the C++ backend parity program links the product library
        hiplib = os.path.join(os.path.dirname(HERE), "pokitlms_amd", "libpokit_hip.so")
        if os.path.exists(hiplib):
            targets += ["cases", "runner"]
    subprocess.run(["make", "-s", "-C", HERE, "-j8", *targets], check=True)


def available(kind: str) -> bool:
    return os.path.exists(PORT_PATH if kind == "port" else REF_PATH)


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what} failed with status {status}")
        self.status = status


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


_ATTENTION_ARGS = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                   ctypes.c_float, ctypes.c_float, _f32p, _f32p, ctypes.c_uint32, _f32p, _f32p,
                   _f32p, _f32p]


class Oracle:
    def __init__(self, kind: str = "port"):
        if kind not in ("port", "reference"):
            raise ValueError(kind)
        self.kind = kind
        path = PORT_PATH if kind == "port" else REF_PATH
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run make -C oracle)")
        self.lib = ctypes.CDLL(path)
        L = self.lib
        if kind == "port":
            L.pko_half_to_float.restype = ctypes.c_float
            L.pko_half_to_float.argtypes = [ctypes.c_uint16]
            L.pko_expf_block_sums.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                              ctypes.c_void_p, ctypes.c_uint32]
            L.pko_expf_block_sums.restype = None
            L.pko_rms_norm.argtypes = [_f32p, _f32p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                       _f32p]
            L.pko_add_rms_norm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_uint64, ctypes.c_uint64,
                                           ctypes.c_float, _f32p]
            L.pko_attention_steps.argtypes = _ATTENTION_ARGS
            L.pko_linear.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64,
                                     ctypes.c_uint64, _f32p, _f32p]
            L.pko_dequantize_row.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p,
                                             ctypes.c_uint64]
            L.pko_route_experts.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int,
                                            _u32p, _f32p, _f32p]
            L.pko_select_experts.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int,
                                             _u32p, _f32p]
            L.pko_moe35_block.argtypes = [
                _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _u8p,
                ctypes.c_uint32, _u8p, ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_int,
                ctypes.c_float, _f32p, ctypes.c_uint32, ctypes.c_uint32, _u8p, ctypes.c_uint32,
                _u8p, ctypes.c_uint32, _u8p, _f32p, _f32p, _u32p, _f32p]
            L.pko_moe_block.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                        ctypes.c_uint32, _u8p, ctypes.c_uint32, _u8p,
                                        ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_int,
                                        _f32p, _f32p, _u32p, _f32p]
        else:
            L.pkref_row_workers.restype = ctypes.c_uint
            L.pkref_rms_norm.argtypes = [_f32p, _f32p, ctypes.c_uint64, ctypes.c_uint64,
                                         ctypes.c_float, _f32p]
            L.pkref_attention_steps.argtypes = _ATTENTION_ARGS
            L.pkref_tensor_linear.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64,
                                              _u8p, ctypes.c_uint64, _f32p, _f32p]
            L.pkref_tensor_linear_repeat.argtypes = [ctypes.c_uint32, ctypes.c_uint64,
                                                     ctypes.c_uint64, _u8p, ctypes.c_uint64,
                                                     _f32p, _f32p, ctypes.c_uint32]
            L.pkref_dequantize_row.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p,
                                               ctypes.c_uint64]
            L.pkref_route_experts.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32,
                                              ctypes.c_int, _u32p, _f32p, _f32p]
            L.pkref_moe_create.restype = ctypes.c_void_p
            L.pkref_moe_create.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.c_uint32, ctypes.c_uint32, _u8p,
                                           ctypes.c_uint32, _u8p, ctypes.c_uint32, _u8p,
                                           ctypes.c_uint32, ctypes.c_int]
            L.pkref_moe_forward.argtypes = [ctypes.c_void_p, _f32p, _f32p, _u32p, _f32p]
            L.pkref_moe_destroy.argtypes = [ctypes.c_void_p]
            L.pkref_qwen3moe_greedy.argtypes = [ctypes.c_char_p, _u32p, ctypes.c_uint32,
                                                ctypes.c_uint32, ctypes.c_uint64, _u32p, _f32p,
                                                ctypes.POINTER(ctypes.c_double)]
            L.pkref_select_experts.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32,
                                               ctypes.c_int, _u32p, _f32p]
            L.pkref_moe35_create.restype = ctypes.c_void_p
            L.pkref_moe35_create.argtypes = [
                _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _u8p,
                ctypes.c_uint32, _u8p, ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_int,
                ctypes.c_float, _f32p, ctypes.c_uint32, ctypes.c_uint32, _u8p, ctypes.c_uint32,
                _u8p, ctypes.c_uint32, _u8p]
            L.pkref_moe35_forward.argtypes = [ctypes.c_void_p, _f32p, _f32p, _u32p, _f32p]
            L.pkref_moe35_destroy.argtypes = [ctypes.c_void_p]
            L.pkref_qwen3moe_forward_times.argtypes = [
                ctypes.c_char_p, _u32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64,
                ctypes.POINTER(ctypes.c_double)]

    # ---- single ops -------------------------------------------------------
    def expf_block_sums(self, first_bits: int, block_size: int, n_blocks: int,
                        threads: int = 16) -> np.ndarray:
        """The host libm's expf as block checksums (pko_expf_block_sums)."""
        out = np.empty(n_blocks, dtype=np.uint64)
        self.lib.pko_expf_block_sums(first_bits, block_size, n_blocks, out.ctypes.data, threads)
        return out

    def half_to_float(self, bits: int) -> float:
        if self.kind != "port":
            raise NotImplementedError("half_to_float is exported by the port only")
        return self.lib.pko_half_to_float(bits)

    def linear(self, gtype: int, weights: np.ndarray, in_features: int, rows: int,
               x: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(weights, dtype=np.uint8)
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        if self.kind == "port":
            rc = self.lib.pko_linear(gtype, w.ctypes.data, w.nbytes, in_features, rows,
                                     _fp(xx), _fp(y))
        else:
            rc = self.lib.pkref_tensor_linear(gtype, in_features, rows, w.ctypes.data, w.nbytes,
                                              _fp(xx), _fp(y))
        if rc:
            raise OracleError(rc, "linear")
        return y

    def linear_repeat(self, gtype, weights, in_features, rows, x, calls) -> np.ndarray:
        """Reference only: ``calls`` tensor_linear calls on one reader (timing)."""
        w = np.ascontiguousarray(weights, dtype=np.uint8)
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        rc = self.lib.pkref_tensor_linear_repeat(gtype, in_features, rows, w.ctypes.data,
                                                 w.nbytes, _fp(xx), _fp(y), calls)
        if rc:
            raise OracleError(rc, "linear_repeat")
        return y

    def rms_norm(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        """rms_norm of each row (src/rms_norm.cpp:9-27)."""
        xx = np.ascontiguousarray(x, dtype=np.float32)
        rows, n = (1, xx.size) if xx.ndim == 1 else xx.shape
        ww = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        out = np.empty_like(xx)
        fn = self.lib.pko_rms_norm if self.kind == "port" else self.lib.pkref_rms_norm
        rc = fn(_fp(xx), _fp(ww), rows, n, float(eps), _fp(out))
        if rc:
            raise OracleError(rc, "rms_norm")
        return out

    def add_rms_norm(self, hidden: np.ndarray, delta, w: np.ndarray, eps: float):
        """Port only: (hidden + delta, rms_norm(hidden + delta, w)) per row."""
        h = np.array(hidden, dtype=np.float32, copy=True)
        rows, n = (1, h.size) if h.ndim == 1 else h.shape
        d = None if delta is None else np.ascontiguousarray(delta, dtype=np.float32)
        ww = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        out = np.empty_like(h)
        rc = self.lib.pko_add_rms_norm(_fp(h), None if d is None else _fp(d), _fp(ww), rows, n,
                                       float(eps), _fp(out))
        if rc:
            raise OracleError(rc, "add_rms_norm")
        return h, out

    def attention_steps(self, heads: int, kv_heads: int, head_dim: int, capacity: int,
                        eps: float, theta: float, q_norm, k_norm, q, k, v) -> np.ndarray:
        """One layer's q/k head norms, RoPE, FP16 KV ring and attention for
        positions 0 .. steps - 1: out [steps][heads * head_dim]."""
        qq = np.ascontiguousarray(q, dtype=np.float32)
        kk = np.ascontiguousarray(k, dtype=np.float32)
        vv = np.ascontiguousarray(v, dtype=np.float32)
        steps = qq.shape[0]
        out = np.zeros((steps, heads * head_dim), np.float32)
        qn = np.ascontiguousarray(q_norm, dtype=np.float32)
        kn = np.ascontiguousarray(k_norm, dtype=np.float32)
        fn = (self.lib.pko_attention_steps if self.kind == "port"
              else self.lib.pkref_attention_steps)
        rc = fn(heads, kv_heads, head_dim, capacity, float(eps), float(theta), _fp(qn), _fp(kn),
                steps, _fp(qq), _fp(kk), _fp(vv), _fp(out))
        if rc:
            raise OracleError(rc, "attention_steps")
        return out

    def dequantize_row(self, gtype: int, encoded: np.ndarray, count: int) -> np.ndarray:
        e = np.ascontiguousarray(encoded, dtype=np.uint8)
        out = np.empty(count, dtype=np.float32)
        fn = self.lib.pko_dequantize_row if self.kind == "port" else self.lib.pkref_dequantize_row
        rc = fn(gtype, e.ctypes.data, e.nbytes, _fp(out), count)
        if rc:
            raise OracleError(rc, "dequantize_row")
        return out

    def route_experts(self, logits: np.ndarray, top_k: int, normalize: bool):
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        ids = np.zeros(max(top_k, 1), dtype=np.uint32)
        sel = np.zeros(max(top_k, 1), dtype=np.float32)
        probs = np.zeros(max(top_k, 1), dtype=np.float32)
        fn = self.lib.pko_route_experts if self.kind == "port" else self.lib.pkref_route_experts
        rc = fn(_fp(lg), lg.size, top_k, int(normalize), ids.ctypes.data_as(_u32p), _fp(sel),
                _fp(probs))
        if rc:
            raise OracleError(rc, "route_experts")
        return ids[:top_k], sel[:top_k], probs[:top_k]

    # ---- MoE block -----------------------------------------------------------
    def qwen3moe_greedy(self, path: str, prompt: np.ndarray, n_new: int,
                        expert_cache_bytes: int = 1 << 40, want_logits: bool = False,
                        vocab: int = 0):
        """The reference Qwen3MoeRunner on a GGUF file (reference library
        only): greedy tokens [n_new], logits after the prompt (or None) and
        the decode forwards' wall seconds."""
        if self.kind != "reference":
            raise OracleError(1, "qwen3moe_greedy needs the compiled reference")
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(n_new, 1), np.uint32)
        logits = np.zeros(vocab, np.float32) if want_logits else None
        secs = ctypes.c_double()
        rc = self.lib.pkref_qwen3moe_greedy(path.encode(), p.ctypes.data_as(_u32p), p.size, n_new,
                                            expert_cache_bytes, out.ctypes.data_as(_u32p),
                                            _fp(logits) if want_logits else None,
                                            ctypes.byref(secs))
        if rc:
            raise OracleError(rc, "pkref_qwen3moe_greedy")
        return out[:n_new], logits, secs.value

    def qwen3moe_forward_times(self, path: str, prompt: np.ndarray, n_forwards: int,
                               expert_cache_bytes: int = 1 << 40) -> np.ndarray:
        """Wall seconds of each of n_forwards greedy decode forwards of the
        reference runner after the prompt (reference library only)."""
        if self.kind != "reference":
            raise OracleError(1, "qwen3moe_forward_times needs the compiled reference")
        p = np.ascontiguousarray(prompt, np.uint32)
        secs = np.zeros(n_forwards, np.float64)
        rc = self.lib.pkref_qwen3moe_forward_times(
            path.encode(), p.ctypes.data_as(_u32p), p.size, n_forwards, expert_cache_bytes,
            secs.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        if rc:
            raise OracleError(rc, "pkref_qwen3moe_forward_times")
        return secs

    def select_experts(self, logits: np.ndarray, top_k: int, normalize: bool):
        """Qwen3.5 select_experts: (ids, weights) in route order."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        ids = np.zeros(max(top_k, 1), dtype=np.uint32)
        w = np.zeros(max(top_k, 1), dtype=np.float32)
        fn = self.lib.pko_select_experts if self.kind == "port" else self.lib.pkref_select_experts
        rc = fn(_fp(lg), lg.size, top_k, int(normalize), ids.ctypes.data_as(_u32p), _fp(w))
        if rc:
            raise OracleError(rc, "select_experts")
        return ids[:top_k], w[:top_k]

    def moe35(self, layer) -> "Moe35Block":
        return Moe35Block(self, layer)

    def moe(self, layer) -> "MoeBlock":
        return MoeBlock(self, layer)


class MoeBlock:
    """A prepared MoE layer; ``forward(x)`` returns (moe_result, ids, probs)."""

    def __init__(self, oracle: Oracle, layer):
        self.o, self.layer = oracle, layer
        self._keep = (np.ascontiguousarray(layer.router, dtype=np.float32),
                      np.ascontiguousarray(layer.gate), np.ascontiguousarray(layer.up),
                      np.ascontiguousarray(layer.down))
        self.handle = None
        if oracle.kind == "reference":
            r, g, u, d = self._keep
            self.handle = oracle.lib.pkref_moe_create(
                _fp(r), layer.hidden, layer.experts, layer.ffn, layer.gate_type, g.ctypes.data,
                layer.up_type, u.ctypes.data, layer.down_type, d.ctypes.data, layer.top_k,
                int(layer.normalize))
            if not self.handle:
                raise OracleError(1, "pkref_moe_create")

    def forward(self, x: np.ndarray):
        L = self.layer
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(L.hidden, dtype=np.float32)
        ids = np.zeros(L.top_k, dtype=np.uint32)
        probs = np.zeros(L.top_k, dtype=np.float32)
        if self.o.kind == "port":
            r, g, u, d = self._keep
            rc = self.o.lib.pko_moe_block(_fp(r), L.hidden, L.experts, L.ffn, L.gate_type,
                                          g.ctypes.data, L.up_type, u.ctypes.data, L.down_type,
                                          d.ctypes.data, L.top_k, int(L.normalize), _fp(xx),
                                          _fp(y), ids.ctypes.data_as(_u32p), _fp(probs))
        else:
            rc = self.o.lib.pkref_moe_forward(self.handle, _fp(xx), _fp(y),
                                              ids.ctypes.data_as(_u32p), _fp(probs))
        if rc:
            raise OracleError(rc, "moe_block")
        return y, ids, probs

    def close(self):
        if self.handle:
            self.o.lib.pkref_moe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Moe35Block:
    """A prepared Qwen3.5-MoE layer (synth.Moe35Layer); ``forward(x)``
    returns (mixer_output, ids, weights)."""

    def __init__(self, oracle: Oracle, layer):
        self.o, self.layer = oracle, layer
        L = layer
        self._keep = tuple(np.ascontiguousarray(a) for a in (
            np.asarray(L.router, np.float32), L.gate, L.up, L.down,
            np.asarray(L.shared_router, np.float32), L.shared_gate, L.shared_up, L.shared_down))
        r, g, u, d, sr, sg, su, sd = self._keep
        self._args = (_fp(r), L.hidden, L.experts, L.ffn, L.gate_type, g.ctypes.data, L.up_type,
                      u.ctypes.data, L.down_type, d.ctypes.data, L.top_k, int(L.normalize),
                      float(L.scale), _fp(sr), L.shared_ffn, L.gate_type, sg.ctypes.data,
                      L.up_type, su.ctypes.data, L.down_type, sd.ctypes.data)
        self.handle = None
        if oracle.kind == "reference":
            self.handle = oracle.lib.pkref_moe35_create(*self._args)
            if not self.handle:
                raise OracleError(1, "pkref_moe35_create")

    def forward(self, x: np.ndarray):
        L = self.layer
        xx = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(L.hidden, np.float32)
        ids = np.zeros(L.top_k, np.uint32)
        w = np.zeros(L.top_k, np.float32)
        if self.handle:
            rc = self.o.lib.pkref_moe35_forward(self.handle, _fp(xx), _fp(y),
                                                ids.ctypes.data_as(_u32p), _fp(w))
        else:
            rc = self.o.lib.pko_moe35_block(*self._args, _fp(xx), _fp(y),
                                            ids.ctypes.data_as(_u32p), _fp(w))
        if rc:
            raise OracleError(rc, "moe35 forward")
        return y, ids, w

    def __del__(self):
        if getattr(self, "handle", None):
            self.o.lib.pkref_moe35_destroy(self.handle)
            self.handle = None
