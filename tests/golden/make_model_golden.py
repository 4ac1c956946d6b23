"""Write tests/golden/model_golden.npz: greedy tokens of the reference
Qwen3MoeRunner on the seeded synthetic Qwen3-MoE models.

Run in a container that has the reference checkout and ~25 GB of free disk:

    make -C oracle ref && python tests/golden/make_model_golden.py [--skip-full]

Each model is written as a GGUF v3 file by pokitlms_amd.synth_model (the same
bytes the GPU generator makes in HBM), loaded by the reference's own
src/gguf_reader.cpp / src/qwen3_moe_index.cpp, and decoded greedily with every
expert held in memory (oracle/_ref/libpkref.so: pkref_qwen3moe_greedy).
Stored per model: shape, seed, prompt, tokens, the reference's decode wall
time, and for the reduced model the logits after the prompt.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, ROOT)

from oracle import Oracle  # noqa: E402
from pokitlms_amd import synth_model as SM  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_golden.npz")

# (tag, layers, prompt tokens, new tokens, keep logits)
MODELS = (("small", 2, 32, 48, True), ("full", 48, 128, 256, False))
SEED = 2024


def shape_for(layers: int) -> SM.Qwen3MoeShape:
    return SM.Qwen3MoeShape(layers=layers)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workdir", default="/tmp/pk_model_golden")
    ap.add_argument("--skip-full", action="store_true")
    args = ap.parse_args()
    os.makedirs(args.workdir, exist_ok=True)
    ref = Oracle("reference")
    out = dict(np.load(OUT, allow_pickle=False)) if os.path.exists(OUT) else {}
    for tag, layers, n_prompt, n_new, keep_logits in MODELS:
        if tag == "full" and args.skip_full:
            continue
        m = shape_for(layers)
        path = os.path.join(args.workdir, f"{tag}.gguf")
        t0 = time.time()
        SM.write_gguf(path, m, SEED)
        print(f"{tag}: wrote {os.path.getsize(path) / 2**30:.2f} GiB in {time.time() - t0:.0f} s",
              flush=True)
        prompt = SM.prompt_tokens(SEED, n_prompt, m.vocab)
        t0 = time.time()
        tokens, logits, decode_s = ref.qwen3moe_greedy(path, prompt, n_new,
                                                       want_logits=keep_logits, vocab=m.vocab)
        print(f"{tag}: reference greedy {n_prompt}+{n_new} in {time.time() - t0:.0f} s "
              f"(decode {decode_s:.1f} s); tokens {tokens[:12]}...", flush=True)
        out[f"{tag}_layers"] = np.array(layers)
        out[f"{tag}_seed"] = np.array(SEED)
        out[f"{tag}_prompt"] = prompt
        out[f"{tag}_tokens"] = tokens
        out[f"{tag}_decode_seconds"] = np.array(decode_s)
        if keep_logits:
            out[f"{tag}_logits"] = logits
        os.remove(path)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
