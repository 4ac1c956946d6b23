"""Write tests/golden/qwen35_golden.npz from the compiled reference CPU path.

Run in a container that has the reference checkout:

    make -C oracle ref && python tests/golden/make_qwen35_golden.py

The vectors come from oracle/_ref/libpkref.so: the reference's select_experts,
silu and sigmoid (src/qwen35_runner.cpp, compiled in place through
oracle/ref_shim35.cpp) and its tensor_linear kernels, composed in the order of
the Qwen3.5-MoE block (src/qwen35_runner.cpp:690-761).  Inputs are regenerated
from seeds by pokitlms_amd.synth; their SHA-256 digests are stored.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, ROOT)

from oracle import Oracle  # noqa: E402
from pokitlms_amd import synth as S  # noqa: E402
from tests.golden.make_golden import route_cases  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen35_golden.npz")

# (name, layer kwargs, tokens): the config-3 widths with a shared expert and a
# route scale, and a narrower layer with other formats and no renormalisation
LAYERS = (
    ("a", dict(seed=35, hidden=2048, experts=128, ffn=768, top_k=8, normalize=True, scale=2.5), 32),
    ("b", dict(seed=36, hidden=1024, experts=64, ffn=512, gate_type=S.Q5_K, up_type=S.Q5_K,
               down_type=S.Q8_0, top_k=6, normalize=False, scale=1.0), 8),
)


def layer_tokens(name, kw, n):
    layer = S.moe35_layer(**kw)
    xs = S.normal_f32(S.rng(kw["seed"] + 100), n * kw["hidden"]).reshape(n, kw["hidden"])
    return layer, xs


def main():
    ref = Oracle("reference")
    out = {}
    for i, (lg, k, norm) in enumerate(route_cases()):
        ids, w = ref.select_experts(lg, k, norm)
        out[f"select{i}_ids"] = ids
        out[f"select{i}_weights"] = w
    for name, kw, n in LAYERS:
        layer, xs = layer_tokens(name, kw, n)
        out[f"{name}_digest"] = np.array(S.digest(
            layer.router, layer.gate, layer.up, layer.down, layer.shared_router,
            layer.shared_gate, layer.shared_up, layer.shared_down, xs))
        blk = ref.moe35(layer)
        ids, ws, ys = [], [], []
        for x in xs:
            y, i, w = blk.forward(x)
            ids.append(i)
            ws.append(w)
            ys.append(y)
        out[f"{name}_ids"] = np.stack(ids)
        out[f"{name}_weights"] = np.stack(ws)
        out[f"{name}_y"] = np.stack(ys[:4])
        out[f"{name}_ysum"] = np.array(S.digest(np.stack(ys)))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
