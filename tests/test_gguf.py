"""GGUF v3 reader/writer (pokitlms_amd/gguf.py) and the seeded model writer
(pokitlms_amd/synth_model.py).

tests/golden/qwen3moe-smoke.gguf is a copy of the reference's data file
tests/data/qwen3moe-smoke.gguf (loaded by its tests/qwen3_moe_smoke_test.cpp),
written by its tools/generate_qwen35_smoke_model.py --architecture qwen3moe:
the metadata and tensor values below are the ones that tool sets
(make_qwen3moe_model), so the reader is checked against a file it did not
write.
"""
import os

import numpy as np
import pytest

from pokitlms_amd import gguf
from pokitlms_amd import synth as S
from pokitlms_amd import synth_model as SM

SMOKE = os.path.join(os.path.dirname(__file__), "golden", "qwen3moe-smoke.gguf")


def _f32(f, name):
    return f.payload(name).view(np.float32)


def test_reads_the_reference_smoke_model():
    with gguf.GgufFile(SMOKE) as f:
        md = f.metadata
        assert md["general.architecture"] == "qwen3moe"
        assert md["general.alignment"] == 32
        expect = {"context_length": 512, "embedding_length": 4, "block_count": 1,
                  "feed_forward_length": 4, "attention.head_count": 1,
                  "attention.head_count_kv": 1, "attention.key_length": 2,
                  "attention.value_length": 2, "rope.dimension_count": 2, "expert_count": 2,
                  "expert_used_count": 1, "expert_feed_forward_length": 2}
        for k, v in expect.items():
            assert md["qwen3moe." + k] == v, k
        assert md["qwen3moe.attention.layer_norm_rms_epsilon"] == np.float32(1e-5)
        assert md["qwen3moe.rope.freq_base"] == 10000.0
        assert md["qwen3moe.tie_word_embeddings"] is False
        assert md["tokenizer.ggml.model"] == "gpt2" and md["tokenizer.ggml.pre"] == "qwen2"
        tokens = md["tokenizer.ggml.tokens"]
        assert len(tokens) == 257 and len(set(tokens)) == 257
        assert list(md["tokenizer.ggml.token_type"]) == [1] * 256 + [3]
        assert md["tokenizer.ggml.bos_token_id"] == md["tokenizer.ggml.eos_token_id"] == 256
        dims = {n: t.dims for n, t in f.tensors.items()}
        assert dims["token_embd.weight"] == [4, 257] and dims["output.weight"] == [4, 257]
        assert dims["blk.0.ffn_gate_exps.weight"] == [4, 2, 2]
        assert dims["blk.0.ffn_down_exps.weight"] == [2, 4, 2]
        assert all(t.gtype == S.F32 for t in f.tensors.values())
        emb = _f32(f, "token_embd.weight").reshape(257, 4)
        assert np.array_equal(emb, np.tile([1.0, 0.0, 0.0, 0.0], (257, 1)).astype(np.float32))
        out = _f32(f, "output.weight").reshape(257, 4)
        want = np.zeros((257, 4), np.float32)
        want[ord("a")] = [1.0, 0.0, 0.0, 0.0]
        assert np.array_equal(out, want)
        for name in ("output_norm.weight", "blk.0.attn_norm.weight", "blk.0.ffn_norm.weight",
                     "blk.0.attn_q_norm.weight", "blk.0.attn_k_norm.weight"):
            assert np.all(_f32(f, name) == 1.0), name
        for name in ("blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight",
                     "blk.0.attn_output.weight", "blk.0.ffn_gate_inp.weight",
                     "blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                     "blk.0.ffn_down_exps.weight"):
            assert np.all(_f32(f, name) == 0.0), name


def test_payload_bytes_of_every_format():
    # rows of 512 elements: 2 super-blocks or 16 32-blocks
    assert gguf.payload_bytes(S.Q4_K, [512, 3]) == 3 * 2 * 144
    assert gguf.payload_bytes(S.Q5_K, [512, 3]) == 3 * 2 * 176
    assert gguf.payload_bytes(S.Q6_K, [512, 3]) == 3 * 2 * 210
    assert gguf.payload_bytes(S.Q8_0, [512, 3]) == 3 * 16 * 34
    assert gguf.payload_bytes(S.Q4_0, [512, 3]) == 3 * 16 * 18
    assert gguf.payload_bytes(S.F32, [512, 3, 2]) == 512 * 3 * 2 * 4


TINY = SM.Qwen3MoeShape(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64, experts=4,
                        top_k=2, ffn=256, vocab=512, context=256)


def test_seeded_writer_round_trip(tmp_path):
    path = str(tmp_path / "tiny.gguf")
    SM.write_gguf(path, TINY, 9)
    with gguf.GgufFile(path) as f:
        assert f.metadata["qwen3moe.block_count"] == 1
        assert f.metadata["qwen3moe.expert_count"] == 4
        assert len(f.metadata["tokenizer.ggml.tokens"]) == 512
        listed = SM.tensor_list(TINY)
        assert list(f.tensors) == [name for name, *_ in listed]
        for i, (name, dims, gtype, kind) in enumerate(listed):
            t = f.tensors[name]
            assert t.dims == dims and t.gtype == gtype
            want = SM.tensor_payload(9, i, gtype, kind, gguf.payload_bytes(gtype, dims))
            assert np.array_equal(f.payload(name), want), name


def test_reference_runner_reads_the_seeded_file(tmp_path):
    """The reference's own GGUF reader and Qwen3MoeRunner accept the file and
    decode greedy tokens from it (oracle/_ref; skipped where it is not built)."""
    import oracle
    if not oracle.available("reference"):
        pytest.skip("oracle/_ref not built")
    path = str(tmp_path / "tiny.gguf")
    SM.write_gguf(path, TINY, 9)
    ref = oracle.Oracle("reference")
    tokens, logits, _ = ref.qwen3moe_greedy(path, SM.prompt_tokens(9, 6, TINY.vocab), 4,
                                            want_logits=True, vocab=TINY.vocab)
    assert tokens.shape == (4,) and np.all(tokens < TINY.vocab)
    assert np.all(np.isfinite(logits)) and int(np.argmax(logits)) == int(tokens[0])
