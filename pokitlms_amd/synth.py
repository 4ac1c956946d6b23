"""Seeded synthetic GGUF-compatible inputs for the routed-MoE K-quant path.

Every generator returns the exact bytes a GGUF file would hold for the tensor
(row-major ``[out, in]`` rows of encoded blocks; expert tensors ``[in, out, E]``
with the expert index slowest), so the same buffers feed the HIP backend and
the CPU checkers.

Randomness: NumPy ``Generator(PCG64(seed))``.  Quant fields are uniform random
bytes; every fp16 scale (``d``, ``dmin``) is ``|N(0, std)|`` rounded to
binary16; activations are ``N(0, 1)`` float32; the F32 router is
``N(0, 0.02)``.  Block layouts follow the reference decoders
(src/quantized_linear.cpp:53-62, 166-205, 286-358, 387-423 of the reference).
"""
from __future__ import annotations

import hashlib

import numpy as np

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 13, 14, 30
Q5_0, Q5_1, Q2_K, Q3_K = 6, 7, 10, 11

TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
              Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K",
              Q6_K: "Q6_K", BF16: "BF16"}
BLOCK_ELEMENTS = {F32: 1, F16: 1, BF16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32,
                  Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, BF16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34,
               Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
# Byte offsets of the fp16 scale fields inside one block.
SCALE_OFFSETS = {Q4_0: (0,), Q4_1: (0, 2), Q5_0: (0,), Q5_1: (0, 2), Q8_0: (0,),
                 Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,)}
# Scale fields stored negative: Q4_1's and Q5_1's m is the block minimum,
# w = q * d + m.
NEGATIVE_SCALES = {Q4_1: (2,), Q5_1: (2,)}


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def row_bytes(gtype: int, in_features: int) -> int:
    be = BLOCK_ELEMENTS[gtype]
    if in_features % be:
        raise ValueError(f"{TYPE_NAMES[gtype]} rows need a multiple of {be} elements")
    return in_features // be * BLOCK_BYTES[gtype]


def matrix_bytes(gtype: int, in_features: int, rows: int) -> int:
    return rows * row_bytes(gtype, in_features)


def half_abs_normal(gen: np.random.Generator, n: int, std: float) -> np.ndarray:
    """``n`` binary16 bit patterns of |N(0, std)| (round to nearest even)."""
    return np.abs(gen.standard_normal(n) * std).astype(np.float16).view(np.uint16)


def normal_f32(gen: np.random.Generator, n: int, std: float = 1.0) -> np.ndarray:
    return (gen.standard_normal(n) * std).astype(np.float32)


def quant_matrix(gtype: int, rows: int, in_features: int, gen: np.random.Generator,
                 scale_std: float = 0.02) -> np.ndarray:
    """Encoded weights, uint8 of shape ``(rows, row_bytes)``.

    Float types are N(0, scale_std) values in that storage type.
    """
    if gtype == F32:
        return normal_f32(gen, rows * in_features, scale_std).view(np.uint8).reshape(rows, -1)
    if gtype == F16:
        vals = (gen.standard_normal(rows * in_features) * scale_std).astype(np.float16)
        return vals.view(np.uint8).reshape(rows, -1)
    if gtype == BF16:
        vals = normal_f32(gen, rows * in_features, scale_std).view(np.uint32)
        return (vals >> 16).astype(np.uint16).view(np.uint8).reshape(rows, -1)
    bb = BLOCK_BYTES[gtype]
    nblocks = rows * (in_features // BLOCK_ELEMENTS[gtype])
    row_bytes(gtype, in_features)  # validates divisibility
    blocks = gen.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    for off in SCALE_OFFSETS[gtype]:
        blocks[:, off:off + 2] = half_abs_normal(gen, nblocks, scale_std).view(np.uint8).reshape(-1, 2)
    for off in NEGATIVE_SCALES.get(gtype, ()):
        blocks[:, off + 1] |= 0x80  # binary16 sign bit
    return blocks.reshape(rows, -1)


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.hexdigest()


class MoeLayer:
    """One Qwen3-MoE MoE layer's routed weights (host copies).

    router: float32 ``(experts, hidden)``; gate/up: ``experts`` slices of a
    ``hidden -> ffn`` matrix; down: ``experts`` slices of ``ffn -> hidden``.
    The expert tensors are uint8 ``(experts, slice_bytes)``, i.e. the GGUF
    ``[in, out, E]`` payload with expert ``e`` at byte ``e * slice_bytes``.
    """

    def __init__(self, router, gate, up, down, hidden, experts, ffn,
                 gate_type=Q4_K, up_type=Q4_K, down_type=Q6_K, top_k=8, normalize=True):
        self.router = router
        self.gate, self.up, self.down = gate, up, down
        self.hidden, self.experts, self.ffn = hidden, experts, ffn
        self.gate_type, self.up_type, self.down_type = gate_type, up_type, down_type
        self.top_k, self.normalize = top_k, normalize

    def routed_bytes(self) -> int:
        """Algorithmic bytes of one single-token pass: router + top_k experts."""
        per_expert = self.gate.shape[1] + self.up.shape[1] + self.down.shape[1]
        return self.router.nbytes + self.top_k * per_expert


def moe_layer(seed: int, hidden: int = 2048, experts: int = 128, ffn: int = 768,
              gate_type: int = Q4_K, up_type: int = Q4_K, down_type: int = Q6_K,
              top_k: int = 8, normalize: bool = True, router_std: float = 0.02) -> MoeLayer:
    gen = rng(seed)
    router = normal_f32(gen, experts * hidden, router_std).reshape(experts, hidden)
    gate = quant_matrix(gate_type, experts * ffn, hidden, gen).reshape(experts, -1)
    up = quant_matrix(up_type, experts * ffn, hidden, gen).reshape(experts, -1)
    down = quant_matrix(down_type, experts * hidden, ffn, gen).reshape(experts, -1)
    return MoeLayer(router, gate, up, down, hidden, experts, ffn, gate_type, up_type,
                    down_type, top_k, normalize)


class Moe35Layer(MoeLayer):
    """A Qwen3.5-MoE layer (src/qwen35_runner.cpp:670-764): the routed
    experts of MoeLayer (``normalize`` = expert_weights_norm, ``scale`` =
    expert_weights_scale) plus the shared expert: ``shared_router`` float32
    ``(hidden,)``, ``shared_gate``/``shared_up`` ``hidden -> shared_ffn`` and
    ``shared_down`` ``shared_ffn -> hidden`` GGUF payloads (uint8)."""

    def __init__(self, base: MoeLayer, scale, shared_router, shared_gate, shared_up,
                 shared_down, shared_ffn):
        super().__init__(base.router, base.gate, base.up, base.down, base.hidden, base.experts,
                         base.ffn, base.gate_type, base.up_type, base.down_type, base.top_k,
                         base.normalize)
        self.scale = scale
        self.shared_router = shared_router
        self.shared_gate, self.shared_up, self.shared_down = shared_gate, shared_up, shared_down
        self.shared_ffn = shared_ffn

    def routed_bytes(self) -> int:
        return (super().routed_bytes() + self.shared_router.nbytes + self.shared_gate.nbytes +
                self.shared_up.nbytes + self.shared_down.nbytes)


def moe35_layer(seed: int, hidden: int = 2048, experts: int = 128, ffn: int = 768,
                gate_type: int = Q4_K, up_type: int = Q4_K, down_type: int = Q6_K,
                top_k: int = 8, normalize: bool = True, scale: float = 1.0,
                router_std: float = 0.02) -> Moe35Layer:
    """Seeded Qwen3.5-MoE layer; the shared expert has the routed experts'
    types and width."""
    base = moe_layer(seed, hidden, experts, ffn, gate_type, up_type, down_type, top_k,
                     normalize, router_std)
    gen = rng(seed + 7919)
    shared_router = normal_f32(gen, hidden, router_std * 10.0)
    sg = quant_matrix(gate_type, ffn, hidden, gen)
    su = quant_matrix(up_type, ffn, hidden, gen)
    sd = quant_matrix(down_type, hidden, ffn, gen)
    return Moe35Layer(base, scale, shared_router, sg, su, sd, ffn)


def dyadic_matrix(gtype: int, rows: int, in_features: int, gen: np.random.Generator) -> np.ndarray:
    """Random quant fields with power-of-two scales (2^-4 or 2^-3).

    Sub-block scales are kept small (K-quant 6-bit fields <= 15, Q6_K int8
    scales in [-8, 7]).  With dyadic activations (``dyadic_vector``) every
    decoded weight, product and partial sum is then a multiple of 2^-8; as
    long as sum |w*x| of a row stays below 2^16 (checked by the tests) every
    partial sum is exact in FP32, so every summation order gives the same
    bits and GPU and CPU results can be compared bit for bit.
    """
    m = quant_matrix(gtype, rows, in_features, gen)
    if gtype in (F32, F16, BF16):
        return m
    blocks = m.reshape(-1, BLOCK_BYTES[gtype])
    for off in SCALE_OFFSETS[gtype]:
        exps = gen.integers(-4, -2, size=blocks.shape[0])
        blocks[:, off:off + 2] = np.ldexp(1.0, exps).astype(np.float16).view(np.uint8).reshape(-1, 2)
    for off in NEGATIVE_SCALES.get(gtype, ()):
        blocks[:, off + 1] |= 0x80
    if gtype == Q6_K:
        blocks[:, 192:208] = (gen.integers(-8, 8, size=(blocks.shape[0], 16))
                              .astype(np.int8).view(np.uint8))
    if gtype in (Q4_K, Q5_K):
        blocks[:, 4:16] &= 0x0F
    if gtype == Q3_K:  # every 6-bit scale 32 + low nibble: scale - 32 in [0, 15]
        blocks[:, 104:108] = 0xAA
    return m


def dyadic_vector(gen: np.random.Generator, n: int) -> np.ndarray:
    """Activations k/16 with k in [-16, 16]."""
    return (gen.integers(-16, 17, size=n).astype(np.float32) / 16.0).astype(np.float32)


# ---- skewed expert load for batched prefill ------------------------------------------

def zipf_targets(tokens: int, experts: int, top_k: int, s: float = 1.1) -> np.ndarray:
    """Expected tokens per expert, by load rank, under Zipf(s): shares
    proportional to rank**-s of the tokens * top_k (token, route) pairs.  A
    token picks distinct experts, so no expert can take more than ``tokens``;
    capped ranks hold exactly ``tokens`` and the rest share what is left in
    the same proportions."""
    w = np.arange(1, experts + 1, dtype=np.float64) ** -s
    total = float(tokens * top_k)
    capped = np.zeros(experts, bool)
    while True:
        t = np.where(capped, float(tokens), 0.0)
        free = ~capped
        t[free] = (total - tokens * capped.sum()) * w[free] / w[free].sum()
        over = free & (t > tokens)
        if not over.any():
            return t
        capped |= over


def zipf_direction(seed: int, hidden: int) -> np.ndarray:
    g = rng(seed)
    u = g.standard_normal(hidden)
    return u / np.linalg.norm(u)


def pin_direction(z: np.ndarray, u: np.ndarray, a: float = 1.0) -> np.ndarray:
    """Tokens N(0, 1) with their component along the unit vector ``u`` set to
    ``a``: every token then shares the term a * (W_e . u) of its router logits,
    while each coordinate stays within |u_i| (about hidden**-0.5) of N(0, 1)."""
    z = np.asarray(z, np.float64)
    return (z - np.outer(z @ u, u) + a * u).astype(np.float32)


def zipf_router(experts: int, hidden: int, top_k: int, seed: int, s: float = 1.1,
                calib_tokens: int = 4096, iters: int = 200) -> tuple[np.ndarray, np.ndarray]:
    """Router rows (float32 [experts, hidden]) that realise a Zipf(s) expert
    load on tokens drawn by ``zipf_tokens(seed, ...)``.

    The reference router is a bias-free matvec (src/qwen3_moe_runner.cpp:
    645-646), so the skew is carried by the rows: W_e = G_e + beta_e * u with
    G_e ~ N(0, 1/hidden) (logit noise of unit variance) and u the tokens'
    pinned direction.  The offsets beta_e are fitted on ``calib_tokens``
    tokens drawn independently of the measured ones, so that expert e's
    share of the top-k selections matches the Zipf target of its load rank;
    ranks are assigned to expert ids in a seeded random order.  Returns the
    router and each expert's target share: its expected picks per token
    (the shares sum to top_k; multiply by a token count for counts)."""
    E, H, K = experts, hidden, top_k
    g = rng(seed + 1)
    u = zipf_direction(seed, H)
    G = g.standard_normal((E, H)) / np.sqrt(H)
    share = zipf_targets(1, E, K, s)               # per token, sums to K
    share = share[g.permutation(E)]                # rank -> expert id
    zc = pin_direction(rng(seed + 2).standard_normal((calib_tokens, H)), u, 0.0)
    noise = zc.astype(np.float64) @ G.T           # [calib, E]
    target = np.clip(share, 1.0 / calib_tokens, 1.0 - 0.5 / calib_tokens)
    bias = np.log(target) * 2.0
    for _ in range(iters):
        logits = noise + bias
        kth = np.partition(logits, E - K, axis=1)[:, E - K][:, None]
        freq = (logits >= kth).mean(axis=0)
        step = np.log(target) - np.log(np.maximum(freq, 0.25 / calib_tokens))
        bias += 0.5 * step
    beta = bias - G @ u                           # a = 1: logit bias = (G_e . u + beta_e)
    W = G + np.outer(beta, u)
    return W.astype(np.float32), share


def zipf_tokens(seed: int, tokens: int, hidden: int) -> np.ndarray:
    """Prefill tokens for ``zipf_router(seed)``: N(0, 1) with the pinned
    direction set to 1."""
    z = rng(seed + 3).standard_normal((tokens, hidden))
    return pin_direction(z, zipf_direction(seed, hidden), 1.0)


def zipf_fit(counts: np.ndarray) -> float:
    """Least-squares Zipf exponent of per-expert counts: minus the slope of
    log(count) against log(rank) over the ranks whose count is nonzero and
    below the largest (capped) count."""
    c = np.sort(np.asarray(counts, np.float64))[::-1]
    r = np.arange(1, c.size + 1, dtype=np.float64)
    keep = (c > 0) & (c < c[0])
    if keep.sum() < 3:
        return float("nan")
    slope = np.polyfit(np.log(r[keep]), np.log(c[keep]), 1)[0]
    return float(-slope)
