"""Write tests/golden/golden.npz from the compiled reference CPU path.

Run in a container that has the reference checkout:

    make -C oracle ref && python tests/golden/make_golden.py

The vectors come from oracle/_ref/libpkref.so, i.e. the reference's own
src/quantized_linear.cpp, src/linear.cpp, src/tensor_linear.cpp and
src/qwen3_moe_runner.cpp (route_experts and the MoE block order) compiled in
place.  Inputs are regenerated from seeds by pokitlms_amd.synth; their SHA-256
digests are stored so a drift in generation fails loudly instead of silently.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, ROOT)

from oracle import Oracle  # noqa: E402
from pokitlms_amd import synth as S  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")

C2_TYPES = (S.Q4_0, S.Q4_1, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K)
C2_SHAPES = ((2048, 6144), (6144, 2048))  # (rows, in) = out x in


def c1_inputs():
    """Config 1: Q4_K 4096x4096, x ~ N(0,1), seed 0."""
    g = S.rng(0)
    w = S.quant_matrix(S.Q4_K, 4096, 4096, g)
    x = S.normal_f32(g, 4096)
    return w, x


def c2_inputs(gtype, rows, inn, batch=8):
    g = S.rng(1000 + gtype * 10 + (rows > inn))
    w = S.quant_matrix(gtype, rows, inn, g)
    xs = S.normal_f32(g, batch * inn).reshape(batch, inn)
    return w, xs


def c3_layer():
    return S.moe_layer(seed=3)


def c3_tokens(n=64):
    g = S.rng(33)
    return S.normal_f32(g, n * 2048).reshape(n, 2048)


def small_inputs(gtype, seed=7, rows=37, inn=512):
    """The reference parity harness shape (tests/vulkan_linear_cases.hpp:31-33)."""
    g = S.rng(seed + gtype)
    inn = 257 if gtype in (S.F32, S.F16, S.BF16) else inn
    return S.quant_matrix(gtype, rows, inn, g), S.normal_f32(g, inn), inn


def route_cases():
    """Random logits plus tie, near-tie and small-count cases."""
    g = S.rng(44)
    cases = []
    for i in range(48):
        cases.append((S.normal_f32(g, 128, 0.9), 8, bool(i % 2)))
    base = S.normal_f32(g, 128, 0.9)
    tied = base.copy()
    tied[10] = tied[20] = tied[30] = np.float32(3.5)  # three-way tie at the top
    cases.append((tied, 8, True))
    near = base.copy()
    near[5] = np.float32(2.75)
    near[6] = np.nextafter(np.float32(2.75), np.float32(0))  # one ulp apart
    cases.append((near, 8, True))
    cases.append((np.zeros(128, np.float32), 8, True))      # all equal: ids 0..7
    cases.append((S.normal_f32(g, 4), 4, False))             # k == n
    cases.append((S.normal_f32(g, 16), 1, True))             # k == 1
    return cases


def main():
    ref = Oracle("reference")
    out = {}
    w, x = c1_inputs()
    out["c1_digest"] = np.array(S.digest(w, x))
    out["c1_y"] = ref.linear(S.Q4_K, w, 4096, 4096, x)

    for t in C2_TYPES:
        for rows, inn in C2_SHAPES:
            w, xs = c2_inputs(t, rows, inn)
            key = f"c2_{S.TYPE_NAMES[t]}_{rows}x{inn}"
            out[key + "_digest"] = np.array(S.digest(w, xs))
            out[key + "_y0"] = ref.linear(t, w, inn, rows, xs[0])
            # Checksum of all 8 outputs, so the full batch is pinned too.
            ys = np.stack([ref.linear(t, w, inn, rows, xs[b]) for b in range(8)])
            out[key + "_ysum"] = np.array(S.digest(ys))

    for t in (S.F32, S.F16, S.BF16, S.Q4_0, S.Q4_1, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K,
              S.Q5_0, S.Q5_1, S.Q2_K, S.Q3_K):
        w, x, inn = small_inputs(t)
        key = f"small_{S.TYPE_NAMES[t]}"
        out[key + "_digest"] = np.array(S.digest(w, x))
        out[key + "_y"] = ref.linear(t, w, inn, 37, x)
        if t not in (S.F32, S.F16, S.BF16):
            out[key + "_row0"] = ref.dequantize_row(t, w[0], inn)

    layer = c3_layer()
    toks = c3_tokens()
    out["c3_digest"] = np.array(S.digest(layer.router, layer.gate, layer.up, layer.down, toks))
    blk = ref.moe(layer)
    ids, probs, ys = [], [], []
    for x in toks:
        y, i, p = blk.forward(x)
        ids.append(i)
        probs.append(p)
        ys.append(y)
    out["c3_ids"] = np.stack(ids)
    out["c3_probs"] = np.stack(probs)
    out["c3_y"] = np.stack(ys[:4])
    out["c3_ysum"] = np.array(S.digest(np.stack(ys)))

    rc = route_cases()
    for i, (lg, k, norm) in enumerate(rc):
        ids, sel, probs = ref.route_experts(lg, k, norm)
        out[f"route{i}_logits"] = lg
        out[f"route{i}_k"] = np.array(k)
        out[f"route{i}_norm"] = np.array(norm)
        out[f"route{i}_ids"] = ids
        out[f"route{i}_probs"] = probs
    out["route_count"] = np.array(len(rc))

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
