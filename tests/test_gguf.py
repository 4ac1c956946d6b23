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


# ---- validation (GgufReader's checks, src/gguf_reader.cpp:173-255) ------------------

def _build(metadata=(), tensors=(), alignment_pad=32, tail=b"", version=3, magic=b"GGUF"):
    """Raw GGUF bytes from explicit fields: metadata [(key, type, payload bytes)],
    tensors [(name, dims, gtype, offset)], the data section padded to
    alignment_pad and followed by `tail`."""
    import struct
    out = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for k, t, payload in metadata:
        out += gguf._str(k) + struct.pack("<I", t) + payload
    for name, dims, gtype, off in tensors:
        out += gguf._str(name) + struct.pack("<I", len(dims))
        out += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", gtype, off)
    out += b"\0" * ((-len(out)) % alignment_pad)
    return bytes(out) + tail


def _u32(v):
    import struct
    return struct.pack("<I", v)


def _parse(tmp_path, raw):
    p = tmp_path / "t.gguf"
    p.write_bytes(raw)
    return gguf.GgufFile(str(p))


F32_4x2 = ("a", [4, 2], S.F32, 0)  # 32 bytes
F32_4x2b = ("b", [4, 2], S.F32, 32)


def test_valid_minimal_file(tmp_path):
    with _parse(tmp_path, _build(tensors=[F32_4x2, F32_4x2b], tail=bytes(64))) as f:
        assert f.alignment == 32 and f.tensors["b"].offset == 32
        assert f.payload("b").size == 32


@pytest.mark.parametrize("raw, message", [
    (b"GGUX" + bytes(60), "magic"),
    (_build(version=2), "version 3"),
    (b"GGUF" + _u32(3), "truncated"),
    (b"", "truncated"),
])
def test_rejects_bad_headers(tmp_path, raw, message):
    with pytest.raises(ValueError, match=message):
        _parse(tmp_path, raw)


def test_rejects_truncated_directory(tmp_path):
    raw = _build(tensors=[F32_4x2], tail=bytes(32))
    for cut in (30, 40, 50):
        with pytest.raises(ValueError, match="truncated|oversized|limits"):
            _parse(tmp_path, raw[:cut])


def test_rejects_payload_past_the_end(tmp_path):
    with pytest.raises(ValueError, match="extends beyond file"):
        _parse(tmp_path, _build(tensors=[F32_4x2, F32_4x2b], tail=bytes(60)))


def test_rejects_overlapping_payloads(tmp_path):
    over = ("b", [4, 2], S.F32, 0)  # same offset as "a"
    with pytest.raises(ValueError, match="overlapping"):
        _parse(tmp_path, _build(tensors=[F32_4x2, over], tail=bytes(64)))
    big = ("a", [8, 2], S.F32, 0)  # 64 bytes reach into "b" at 32
    with pytest.raises(ValueError, match="overlapping"):
        _parse(tmp_path, _build(tensors=[big, F32_4x2b], tail=bytes(96)))


def test_rejects_misaligned_offset(tmp_path):
    with pytest.raises(ValueError, match="data offset"):
        _parse(tmp_path, _build(tensors=[("a", [4, 2], S.F32, 8)], tail=bytes(64)))


def test_rejects_duplicate_names_and_keys(tmp_path):
    dup = ("a", [4, 2], S.F32, 32)
    with pytest.raises(ValueError, match="duplicate GGUF tensor name"):
        _parse(tmp_path, _build(tensors=[F32_4x2, dup], tail=bytes(64)))
    md = [("k", gguf.U32, _u32(1)), ("k", gguf.U32, _u32(2))]
    with pytest.raises(ValueError, match="duplicate GGUF metadata key"):
        _parse(tmp_path, _build(metadata=md))


@pytest.mark.parametrize("t, v, ok", [(gguf.U32, 0, False), (gguf.U32, 12, False),
                                      (gguf.U32, 4, False), (gguf.I32, 32, False),
                                      (gguf.U32, 24, True), (gguf.U64, 64, True)])
def test_alignment_rules(tmp_path, t, v, ok):
    import struct
    payload = struct.pack("<i" if t == gguf.I32 else ("<Q" if t == gguf.U64 else "<I"), v)
    raw = _build(metadata=[("general.alignment", t, payload)], tensors=[F32_4x2],
                 alignment_pad=v if ok else 32, tail=bytes(64))
    if ok:
        with _parse(tmp_path, raw) as f:
            assert f.alignment == v
    else:
        with pytest.raises(ValueError, match="alignment"):
            _parse(tmp_path, raw)


def test_rejects_bad_tensor_shapes(tmp_path):
    with pytest.raises(ValueError, match="rank"):
        _parse(tmp_path, _build(tensors=[("a", [], S.F32, 0)], tail=bytes(32)))
    with pytest.raises(ValueError, match="zero-sized"):
        _parse(tmp_path, _build(tensors=[("a", [4, 0], S.F32, 0)], tail=bytes(32)))
    with pytest.raises(ValueError, match="multiple of 256"):
        _parse(tmp_path, _build(tensors=[("a", [100, 1], S.Q4_K, 0)], tail=bytes(256)))


def test_rejects_bad_metadata_values(tmp_path):
    with pytest.raises(ValueError, match="boolean"):
        _parse(tmp_path, _build(metadata=[("b", gguf.BOOL, b"\x02")]))
    with pytest.raises(ValueError, match="value type"):
        _parse(tmp_path, _build(metadata=[("x", 13, _u32(0))]))
    import struct
    huge = struct.pack("<Q", 1 << 40)
    with pytest.raises(ValueError, match="oversized GGUF string"):
        _parse(tmp_path, _build(metadata=[("s", gguf.STRING, huge)]))
    arr = struct.pack("<IQ", gguf.U8, 1 << 40)
    with pytest.raises(ValueError, match="oversized GGUF array"):
        _parse(tmp_path, _build(metadata=[("a", gguf.ARRAY, arr)]))


def test_unknown_tensor_type_parses_but_has_no_payload(tmp_path):
    """A type without a known layout parses, as in the reference (its payload
    size is unknown there), and its payload is refused."""
    with _parse(tmp_path, _build(tensors=[("a", [4, 2], 99, 0), F32_4x2b], tail=bytes(64))) as f:
        assert f.tensors["a"].gtype == 99 and not f.tensors["a"].known_layout
        with pytest.raises(ValueError, match="no known block layout"):
            f.payload("a")
        assert f.payload("b").size == 32


def test_reference_data_files_parse():
    """Every GGUF file the reference ships under tests/data parses (the Q/K/V
    smoke models; skipped where the reference checkout is absent)."""
    import glob
    files = sorted(glob.glob("/root/reference/tests/data/*.gguf"))
    if not files:
        pytest.skip("reference checkout absent")
    for path in files:
        with gguf.GgufFile(path) as f:
            assert f.tensors and all(t.known_layout for t in f.tensors.values())
