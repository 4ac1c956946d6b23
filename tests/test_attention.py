"""Pins the oracle's attention stage (pko_attention_steps) and residual-add
RMSNorm (pko_add_rms_norm) before the GPU kernels are compared with them.

* against the reference's own rms_norm, prepare_qwen_rope / apply_qwen_rope
  and FP16 KvCache::append / attend (oracle/_ref, compiled from
  /root/reference/src), bit for bit, at several head layouts, ring windows
  that wrap and the config-5 shape;
* closed forms that hold whatever the rotation: a single position attends to
  its own value (softmax of one score is exactly 1), and a zero query gives
  every cached position the same score, so the output is the window's FP16
  values averaged with weights 1/size summed in window order.
"""
import numpy as np
import pytest

import oracle

CASES = (  # heads, kv_heads, head_dim, capacity, steps
    (8, 2, 128, 16, 40),      # the ring wraps twice
    (32, 4, 128, 512, 24),    # config-5 heads, window not yet full
    (4, 4, 64, 8, 12),        # one q head per kv head
    (6, 2, 256, 5, 9),
)


def _inputs(seed, heads, kv_heads, head_dim, steps, scale=1.0):
    g = np.random.default_rng(seed)
    q = (g.standard_normal((steps, heads * head_dim)) * scale).astype(np.float32)
    k = (g.standard_normal((steps, kv_heads * head_dim)) * 3 * scale).astype(np.float32)
    v = g.standard_normal((steps, kv_heads * head_dim)).astype(np.float32)
    qn = (1 + 0.1 * g.random(head_dim)).astype(np.float32)
    kn = (1 + 0.1 * g.random(head_dim)).astype(np.float32)
    return qn, kn, q, k, v


@pytest.mark.skipif(not oracle.available("reference"), reason="oracle/_ref not built")
@pytest.mark.parametrize("case", CASES)
def test_attention_oracle_equals_reference(port, case):
    heads, kv_heads, head_dim, capacity, steps = case
    ref = oracle.Oracle("reference")
    for seed, scale in ((1, 1.0), (2, 40.0)):  # large scores: the softmax max matters
        args = _inputs(seed, heads, kv_heads, head_dim, steps, scale)
        a = port.attention_steps(heads, kv_heads, head_dim, capacity, 1e-6, 1e6, *args)
        b = ref.attention_steps(heads, kv_heads, head_dim, capacity, 1e-6, 1e6, *args)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (case, seed)


def test_attention_single_position_is_its_value(port):
    heads, kv_heads, head_dim = 8, 2, 128
    qn, kn, q, k, v = _inputs(3, heads, kv_heads, head_dim, 1)
    out = port.attention_steps(heads, kv_heads, head_dim, 4, 1e-6, 1e6, qn, kn, q, k, v)
    want = np.repeat(v.astype(np.float16).astype(np.float32).reshape(kv_heads, head_dim),
                     heads // kv_heads, axis=0).reshape(-1)
    assert np.array_equal(out[0], want)


@pytest.mark.parametrize("capacity", (5, 64))
def test_attention_zero_query_averages_the_window(port, capacity):
    """q = 0 normalises to 0, so every score is 0, every weight exp(0) / size."""
    heads, kv_heads, head_dim, steps = 4, 2, 64, 11
    qn, kn, _, k, v = _inputs(4, heads, kv_heads, head_dim, steps)
    q = np.zeros((steps, heads * head_dim), np.float32)
    out = port.attention_steps(heads, kv_heads, head_dim, capacity, 1e-6, 1e6, qn, kn, q, k, v)
    vh = v.astype(np.float16).astype(np.float32)
    for t in range(steps):
        size = min(t + 1, capacity)
        p = np.float32(1.0) / np.float32(size)
        acc = np.zeros(kv_heads * head_dim, np.float32)
        for i in range(t + 1 - size, t + 1):
            acc = (acc + p * vh[i]).astype(np.float32)
        want = np.repeat(acc.reshape(kv_heads, head_dim), heads // kv_heads, axis=0).reshape(-1)
        assert np.array_equal(out[t], want), t


def test_add_rms_norm_oracle(port):
    g = np.random.default_rng(5)
    h = g.standard_normal((3, 2048)).astype(np.float32)
    d = g.standard_normal((3, 2048)).astype(np.float32)
    w = (1 + 0.1 * g.random(2048)).astype(np.float32)
    hs, out = port.add_rms_norm(h, d, w, 1e-6)
    assert np.array_equal(hs, h + d)
    assert np.array_equal(out.view(np.uint32), port.rms_norm(h + d, w, 1e-6).view(np.uint32))
    hs0, out0 = port.add_rms_norm(h, None, w, 1e-6)
    assert np.array_equal(hs0, h)
    assert np.array_equal(out0.view(np.uint32), port.rms_norm(h, w, 1e-6).view(np.uint32))
