"""Whole-model Qwen3-MoE greedy decode on the HIP backend.

``Qwen3MoeModel`` mirrors Qwen3MoeRunner (include/pokitlms/model/
qwen3_moe_runner.hpp:57-110) for the greedy path: every tensor resident in
HBM (no expert cache), every layer of a token step on the GPU, one captured
HIP graph replayed per token (pk_hip_qwen3moe_* in include/pokit_hip.h).
``reference_order`` (default) runs the kernels that repeat the CPU's
operation order, so greedy tokens follow the reference through near-ties;
False selects the bandwidth-optimised kernels.  Reference order also needs
the host libm's expf exceptions (``libm_expf.bin``, written at build time by
host/expf_table.c), so the device's float exponentials return glibc's bits.

Two ways to build one:
* ``from_gguf(backend, path)``: a GGUF v3 qwen3moe file, tensor names and
  config keys as the reference index reads them (src/qwen3_moe_index.cpp:
  37-85, src/architecture.cpp:59-120), payloads uploaded from the memory-mapped
  file;
* ``synthetic(backend, shape, seed)``: the seeded model of
  pokitlms_amd/synth_model.py generated directly in HBM (pk_hip_synth_weight),
  byte-identical to the GGUF file ``synth_model.write_gguf`` writes.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from pokitlms_amd import _abi
from pokitlms_amd import gguf
from pokitlms_amd import synth as S
from pokitlms_amd import synth_model as SM
from pokitlms_amd.backend import HipBackend, Weight, _ERRBUF, _raise

_LAYER_FIELDS = ("attn_norm", "q", "q_norm", "k", "k_norm", "v", "o", "ffn_norm", "router",
                 "gate", "up", "down")
_LAYER_TENSORS = ("attn_norm", "attn_q", "attn_q_norm", "attn_k", "attn_k_norm", "attn_v",
                  "attn_output", "ffn_norm", "ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps",
                  "ffn_down_exps")


_EXPF_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libm_expf.bin")
_expf_pairs: np.ndarray | None = None


def libm_expf_pairs() -> np.ndarray:
    """uint32 [n, 2] (input bits, libm expf bits), increasing inputs: the
    floats on which the host libm's expf is not the correctly rounded value."""
    global _expf_pairs
    if _expf_pairs is None:
        if not os.path.exists(_EXPF_TABLE):
            raise ImportError(f"{_EXPF_TABLE} missing: run pokitlms_amd.build first")
        raw = np.fromfile(_EXPF_TABLE, dtype=np.uint8)
        if raw.size < 12 or bytes(raw[:8]) != b"PKEXPF01":
            raise ValueError(f"{_EXPF_TABLE}: not an expf exception table")
        n = int(raw[8:12].view(np.uint32)[0])
        if raw.size != 12 + 8 * n:
            raise ValueError(f"{_EXPF_TABLE}: truncated")
        _expf_pairs = raw[12:].view(np.uint32).reshape(n, 2)
    return _expf_pairs


def _upload_args(dims: list[int]) -> tuple[int, int, int]:
    """(in, out, n_experts) of a GGUF tensor for pk_hip_upload."""
    if len(dims) == 1:
        return dims[0], 1, 0
    if len(dims) == 2:
        return dims[0], dims[1], 0
    return dims[0], dims[1], dims[2]


class Qwen3MoeModel:
    def __init__(self, backend: HipBackend, shape: SM.Qwen3MoeShape, weights: dict[str, Weight],
                 reference_order: bool = True):
        self.backend, self.shape, self.weights = backend, shape, weights
        self.reference_order = reference_order
        m = shape
        # the runner's default KV window: min(context, 512) (src/qwen3_moe_runner.cpp:372-376)
        cfg = _abi.Qwen3MoeConfig(m.layers, m.hidden, m.heads, m.kv_heads, m.head_dim, m.experts,
                                  m.top_k, m.ffn, m.vocab, min(m.context, 512), m.context,
                                  1 if m.normalize else 0, 1 if reference_order else 0,
                                  m.rms_eps, m.rope_theta)
        if reference_order:
            pairs = libm_expf_pairs()
            cfg.libm_expf_pairs = pairs.ctypes.data
            cfg.libm_expf_count = pairs.shape[0]
        layers = (_abi.Qwen3MoeLayer * m.layers)()
        for l in range(m.layers):
            for field, name in zip(_LAYER_FIELDS, _LAYER_TENSORS):
                setattr(layers[l], field, weights[f"blk.{l}.{name}.weight"].handle)
        self._layers = layers  # kept alive for the create call
        wts = _abi.Qwen3MoeWeights(weights["token_embd.weight"].handle,
                                   weights["output_norm.weight"].handle,
                                   weights["output.weight"].handle, layers)
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(_ERRBUF)
        _raise(_abi.lib().pk_hip_qwen3moe_create(backend.handle, ctypes.byref(cfg), ctypes.byref(wts),
                                                 ctypes.byref(h), err, _ERRBUF), err)
        self.handle = h.value

    # ---- construction ---------------------------------------------------------------
    @staticmethod
    def synthetic_weights(backend: HipBackend, shape: SM.Qwen3MoeShape,
                          seed: int) -> dict[str, Weight]:
        """Every tensor of the seeded model, generated in HBM, by GGUF name."""
        weights = {}
        L = _abi.lib()
        try:
            for i, (name, dims, gtype, kind) in enumerate(SM.tensor_list(shape)):
                inn, out, ne = _upload_args(dims)
                h = ctypes.c_void_p()
                err = ctypes.create_string_buffer(_ERRBUF)
                _raise(L.pk_hip_synth_weight(backend.handle, gtype, inn, out, ne,
                                             SM.tensor_key(seed, i), kind, ctypes.byref(h), err,
                                             _ERRBUF), err)
                weights[name] = Weight(backend, h.value, gtype, inn, out, ne,
                                       gguf.payload_bytes(gtype, dims))
            return weights
        except BaseException:
            for w in weights.values():
                w.release()
            raise

    @classmethod
    def synthetic(cls, backend: HipBackend, shape: SM.Qwen3MoeShape, seed: int,
                  reference_order: bool = True) -> "Qwen3MoeModel":
        weights = cls.synthetic_weights(backend, shape, seed)
        try:
            return cls(backend, shape, weights, reference_order)
        except BaseException:
            for w in weights.values():
                w.release()
            raise

    @classmethod
    def from_gguf(cls, backend: HipBackend, path: str,
                  reference_order: bool = True) -> "Qwen3MoeModel":
        with gguf.GgufFile(path) as f:
            md = f.metadata
            if md.get("general.architecture") != "qwen3moe":
                raise ValueError("not a qwen3moe GGUF file")
            a = "qwen3moe."
            heads = int(md[a + "attention.head_count"])
            hidden = int(md[a + "embedding_length"])
            shape = SM.Qwen3MoeShape(
                layers=int(md[a + "block_count"]), hidden=hidden, heads=heads,
                kv_heads=int(md.get(a + "attention.head_count_kv", heads)),
                head_dim=int(md.get(a + "attention.key_length", hidden // heads)),
                experts=int(md[a + "expert_count"]), top_k=int(md[a + "expert_used_count"]),
                ffn=int(md[a + "expert_feed_forward_length"]),
                vocab=len(md["tokenizer.ggml.tokens"]), context=int(md[a + "context_length"]),
                rms_eps=float(md[a + "attention.layer_norm_rms_epsilon"]),
                rope_theta=float(md[a + "rope.freq_base"]),
                normalize=bool(md.get(a + "expert_weights_norm", False)),
                attn_type=f.tensors["blk.0.attn_q.weight"].gtype,
                embd_type=f.tensors["token_embd.weight"].gtype,
                out_type=f.tensors.get("output.weight", f.tensors["token_embd.weight"]).gtype,
                gate_type=f.tensors["blk.0.ffn_gate_exps.weight"].gtype,
                down_type=f.tensors["blk.0.ffn_down_exps.weight"].gtype)
            weights = {}
            try:
                for name, t in f.tensors.items():
                    inn, out, ne = _upload_args(t.dims)
                    weights[name] = backend.upload(t.gtype, inn, out, f.payload(name), ne)
                if "output.weight" not in weights:  # tied embeddings (architecture.cpp:101-103)
                    t = f.tensors["token_embd.weight"]
                    weights["output.weight"] = backend.upload(t.gtype, t.dims[0], t.dims[1],
                                                              f.payload("token_embd.weight"))
                return cls(backend, shape, weights, reference_order)
            except BaseException:
                for w in weights.values():
                    w.release()
                raise

    # ---- use --------------------------------------------------------------------------
    def generate(self, prompt: np.ndarray, n_new: int, want_logits: bool = False):
        """Greedy tokens (uint32 [n_new]); the logits after the last prompt
        token (or None); GenerationStats as a dict."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(n_new, 1), np.uint32)
        logits = np.zeros(self.shape.vocab, np.float32) if want_logits else None
        st = _abi.GenerationStats()
        err = ctypes.create_string_buffer(_ERRBUF)
        up = ctypes.POINTER(ctypes.c_uint32)
        _raise(_abi.lib().pk_hip_qwen3moe_generate(
            self.handle, p.ctypes.data_as(up), p.size, n_new, out.ctypes.data_as(up),
            logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if want_logits else None,
            ctypes.byref(st), err, _ERRBUF), err)
        stats = {k: getattr(st, k) for k, _ in st._fields_}
        return out[:n_new], logits, stats

    def resident_bytes(self) -> int:
        return sum(w.nbytes for w in self.weights.values())

    def close(self) -> None:
        if self.handle:
            _abi.lib().pk_hip_qwen3moe_destroy(self.handle)
            self.handle = None
        for w in self.weights.values():
            w.release()
        self.weights = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
