"""Seeded synthetic Qwen3-MoE model (the whole-model decode workload).

Every tensor payload is a pure function of (seed, tensor index): a byte stream
of 64-bit words ``mix(key + i)`` (the splitmix64 output function, little
endian), followed by a per-format fix-up of the scale fields that uses only
integer operations on the stream's own bytes.  The same bytes therefore come
out of NumPy here (``tensor_payload``, used to write a GGUF file for the CPU
reference) and out of the device generator ``pk_hip_synth_fill`` (used to
build the model directly in HBM on the GPU), with no file transfer.

Fix-ups (value ranges chosen to keep 48 residual layers finite and the
softmaxes well spread):
* Q4_K/Q5_K: d = dmin = fp16 bits ((5 + (b1 >> 7)) << 10) | (b1 & 3) << 8 | b0
  from d's two bytes, i.e. [2^-10, 2^-8); sub-block scales sc_j = 1 + (byte
  4 + j & 7) and mins m_j = (15 sc_j + 1) >> 1 (about 7.5 sc_j), packed into the
  12 scale bytes, so each sub-block's weights d (sc_j q - m_j) are centred on
  zero like a trained model's; quants stay uniform.
* Q6_K: fp16 d = ((1 + (b1 >> 7)) << 10) | (b1 & 3) << 8 | b0, i.e. [2^-14,
  2^-12); int8 scales and quants stay uniform (already centred).
* F32 norm weights: 1 + m * 2^-23 with m the low 20 bits (in [1, 1.125)).
* F32 router: sign and 23 mantissa bits random, exponent 2^-7 (|w| in [2^-7, 2^-6)).

Tensor order, names and GGUF dims follow the reference index
(src/qwen3_moe_index.cpp:37-85) and its config keys
(src/architecture.cpp:59-120).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from pokitlms_amd import gguf
from pokitlms_amd import synth as S

GOLDEN_GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

# fix-up kinds (shared with the device generator)
KIND_RAW, KIND_KQUANT, KIND_Q6K, KIND_NORM, KIND_ROUTER = 0, 1, 2, 3, 4


def mix(z: np.ndarray) -> np.ndarray:
    """splitmix64 output for state z (uint64 array, wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = z + GOLDEN_GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def tensor_key(seed: int, index: int) -> int:
    k = mix(np.array([seed], np.uint64))[0] ^ np.uint64(index)
    return int(mix(np.array([k], np.uint64))[0])


@dataclass(frozen=True)
class Qwen3MoeShape:
    layers: int = 48
    hidden: int = 2048
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = 128
    experts: int = 128
    top_k: int = 8
    ffn: int = 768
    vocab: int = 151936
    context: int = 4096
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    normalize: bool = True
    attn_type: int = S.Q4_K
    embd_type: int = S.Q4_K
    out_type: int = S.Q6_K
    gate_type: int = S.Q4_K
    down_type: int = S.Q6_K


def kind_of(gtype: int, role: str) -> int:
    if gtype in (S.Q4_K, S.Q5_K):
        return KIND_KQUANT
    if gtype == S.Q6_K:
        return KIND_Q6K
    if gtype == S.F32:
        return KIND_ROUTER if role == "router" else KIND_NORM
    raise ValueError(f"no synthetic recipe for type {gtype}")


def tensor_list(m: Qwen3MoeShape) -> list[tuple[str, list[int], int, int]]:
    """(name, GGUF dims, type, fix-up kind) in file order; the index in this
    list is the tensor's generator index."""
    qd, kd = m.heads * m.head_dim, m.kv_heads * m.head_dim
    out = [("token_embd.weight", [m.hidden, m.vocab], m.embd_type, kind_of(m.embd_type, ""))]
    for l in range(m.layers):
        p = f"blk.{l}."
        out += [
            (p + "attn_norm.weight", [m.hidden], S.F32, KIND_NORM),
            (p + "attn_q.weight", [m.hidden, qd], m.attn_type, kind_of(m.attn_type, "")),
            (p + "attn_q_norm.weight", [m.head_dim], S.F32, KIND_NORM),
            (p + "attn_k.weight", [m.hidden, kd], m.attn_type, kind_of(m.attn_type, "")),
            (p + "attn_k_norm.weight", [m.head_dim], S.F32, KIND_NORM),
            (p + "attn_v.weight", [m.hidden, kd], m.attn_type, kind_of(m.attn_type, "")),
            (p + "attn_output.weight", [qd, m.hidden], m.attn_type, kind_of(m.attn_type, "")),
            (p + "ffn_norm.weight", [m.hidden], S.F32, KIND_NORM),
            (p + "ffn_gate_inp.weight", [m.hidden, m.experts], S.F32, KIND_ROUTER),
            (p + "ffn_gate_exps.weight", [m.hidden, m.ffn, m.experts], m.gate_type,
             kind_of(m.gate_type, "")),
            (p + "ffn_up_exps.weight", [m.hidden, m.ffn, m.experts], m.gate_type,
             kind_of(m.gate_type, "")),
            (p + "ffn_down_exps.weight", [m.ffn, m.hidden, m.experts], m.down_type,
             kind_of(m.down_type, "")),
        ]
    out += [("output_norm.weight", [m.hidden], S.F32, KIND_NORM),
            ("output.weight", [m.hidden, m.vocab], m.out_type, kind_of(m.out_type, ""))]
    return out


def _fp16_scale(b0: np.ndarray, b1: np.ndarray, exp: int) -> tuple[np.ndarray, np.ndarray]:
    bits = ((exp + (b1.astype(np.uint16) >> 7)) << 10) | ((b1.astype(np.uint16) & 3) << 8) | b0
    return (bits & 0xFF).astype(np.uint8), (bits >> 8).astype(np.uint8)


def _kquant_scales(r: np.ndarray) -> np.ndarray:
    """12 packed scale/min bytes from the 12 random bytes r (rows of blocks):
    sc_j = 1 + (r[j] & 7), m_j = (15 sc_j + 1) >> 1, in the K-quant 6-bit
    packing (src/quantized_linear.cpp:176-188)."""
    sc = 1 + (r[:, 0:8].astype(np.uint16) & 7)
    m = (15 * sc + 1) >> 1
    q = np.zeros_like(r)
    q[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    q[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    q[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return q


def tensor_payload(seed: int, index: int, gtype: int, kind: int, nbytes: int) -> np.ndarray:
    """The tensor's bytes (uint8, length nbytes)."""
    key = np.uint64(tensor_key(seed, index))
    words = mix(key + np.arange((nbytes + 7) // 8, dtype=np.uint64))
    b = words.view(np.uint8)[:nbytes].copy()
    if kind == KIND_KQUANT:
        blk = b.reshape(-1, S.BLOCK_BYTES[gtype])
        blk[:, 0], blk[:, 1] = _fp16_scale(blk[:, 0], blk[:, 1], 5)
        blk[:, 2], blk[:, 3] = blk[:, 0], blk[:, 1]
        blk[:, 4:16] = _kquant_scales(blk[:, 4:16])
    elif kind == KIND_Q6K:
        blk = b.reshape(-1, 210)
        blk[:, 208], blk[:, 209] = _fp16_scale(blk[:, 208], blk[:, 209], 1)
    elif kind == KIND_NORM:
        u = b.view(np.uint32)
        u[:] = np.uint32(0x3F800000) | (u & np.uint32(0x000FFFFF))
    elif kind == KIND_ROUTER:
        u = b.view(np.uint32)
        u[:] = (u & np.uint32(0x807FFFFF)) | np.uint32(120 << 23)
    return b


def prompt_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    """n uniform token ids (splitmix64 words of a dedicated key, mod vocab)."""
    key = np.uint64(tensor_key(seed, 0xFFFF_FFFF))
    w = mix(key + np.arange(n, dtype=np.uint64))
    return (w % np.uint64(vocab)).astype(np.uint32)


def byte_to_unicode() -> list[str]:
    """GPT-2 byte-level symbols in byte order (the tokenizer's base tokens)."""
    keep = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    out, extra = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return [out[b] for b in range(256)]


def write_gguf(path: str, m: Qwen3MoeShape, seed: int, progress=None) -> None:
    """The seeded model as a GGUF v3 file the reference loads (qwen3moe
    architecture, gpt2/qwen2 tokenizer with the 256 byte tokens and unique
    filler tokens, no merges).  progress(done, total), if given, is called
    after each tensor's payload is made."""
    w = gguf.GgufWriter()
    md = w.metadata
    md["general.architecture"] = "qwen3moe"
    md["general.name"] = "pokitlms-synthetic-qwen3moe"
    a = "qwen3moe."
    md[a + "context_length"] = m.context
    md[a + "embedding_length"] = m.hidden
    md[a + "block_count"] = m.layers
    md[a + "feed_forward_length"] = m.ffn * m.top_k
    md[a + "attention.head_count"] = m.heads
    md[a + "attention.head_count_kv"] = m.kv_heads
    md[a + "attention.key_length"] = m.head_dim
    md[a + "attention.value_length"] = m.head_dim
    md[a + "rope.freq_base"] = float(m.rope_theta)
    md[a + "attention.layer_norm_rms_epsilon"] = float(m.rms_eps)
    md[a + "expert_count"] = m.experts
    md[a + "expert_used_count"] = m.top_k
    md[a + "expert_feed_forward_length"] = m.ffn
    md[a + "expert_weights_norm"] = bool(m.normalize)
    md["tokenizer.ggml.model"] = "gpt2"
    md["tokenizer.ggml.pre"] = "qwen2"
    base = byte_to_unicode()
    tokens = base + [f"<|pk{i}|>" for i in range(m.vocab - len(base))]
    md["tokenizer.ggml.tokens"] = ("array", tokens)
    md["tokenizer.ggml.token_type"] = ("array", np.ones(m.vocab, np.int32))
    md["tokenizer.ggml.merges"] = ("array", [])
    md["tokenizer.ggml.bos_token_id"] = m.vocab - 1
    md["tokenizer.ggml.eos_token_id"] = m.vocab - 2
    items = tensor_list(m)

    def payload(i, gtype, kind, nbytes):
        data = tensor_payload(seed, i, gtype, kind, nbytes)
        if progress is not None:
            progress(i + 1, len(items))
        return data

    for i, (name, dims, gtype, kind) in enumerate(items):
        nbytes = gguf.payload_bytes(gtype, dims)
        w.add_tensor(name, dims, gtype,
                     lambda i=i, gtype=gtype, kind=kind, nbytes=nbytes: payload(i, gtype, kind, nbytes))
    w.write(path)
