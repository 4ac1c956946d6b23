"""The fast decode mode's own kernels against the oracle, at the config-5
shapes (hidden 2048, 32 q heads / 4 kv heads of 128, Q4_K attention rows):

* the residual add + RMSNorm kernel (k_add_rmsnorm4 / k_add_rmsnorm):
  the updated residual bit for bit, the normed row within 1e-4 normwise of
  the reference's rms_norm (pko_add_rms_norm, pinned to src/rms_norm.cpp);
* the fused q/k/v projection: the q, k and v rows of one layer back to back
  as one 5,120-row matrix in one matvec launch, each part within 1e-4 of the
  oracle's tensor_linear on that part;
* the same projection with the residual add and attention RMSNorm in its
  staging (pk_hip_matvec_add_rmsnorm): the residual bit for bit, the
  projection within 1e-4 of tensor_linear on pko_add_rms_norm's row;
* the attention stage (q/k head norms, RoPE, FP16 KV ring, attention): the
  fast kernel within 1e-4 normwise of pko_attention_steps (pinned bit for bit
  to the reference's KvCache::attend) at every position, the reference-order
  kernel bit for bit.
"""
import numpy as np
import pytest

from pokitlms_amd import synth as S
from tests.conftest import normwise_rel

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("n", (2048, 4096, 1000, 8192, 12))
def test_add_rmsnorm_kernel(hip, port, n):
    g = np.random.default_rng(n)
    rows = 3
    h = g.standard_normal((rows, n)).astype(np.float32) * 4
    d = g.standard_normal((rows, n)).astype(np.float32)
    w = (1 + 0.125 * g.random(n)).astype(np.float32)
    for delta in (d, None):
        gh, gout = hip.add_rmsnorm(h, delta, w, 1e-6)
        ch, cout = port.add_rms_norm(h, delta, w, 1e-6)
        assert np.array_equal(gh.view(np.uint32), ch.view(np.uint32))
        err = max(normwise_rel(gout[r], cout[r]) for r in range(rows))
        say("add_rmsnorm n", n, "delta", delta is not None, "normwise", err)
        assert err <= 1e-4, err


@pytest.mark.parametrize("gtype", (S.Q4_K, S.Q5_K, S.Q6_K, S.Q8_0))
def test_fused_qkv_projection(hip, port, gtype):
    hidden, qd, kd = 2048, 4096, 512
    g = S.rng(300 + gtype)
    parts = [S.quant_matrix(gtype, rows, hidden, g) for rows in (qd, kd, kd)]
    x = S.normal_f32(g, hidden)
    w = hip.upload(gtype, hidden, qd + 2 * kd, np.concatenate(parts))
    try:
        y = hip.matvec(w, x)
    finally:
        w.release()
    off = 0
    for name, rows, enc in zip("qkv", (qd, kd, kd), parts):
        want = port.linear(gtype, enc, hidden, rows, x)
        err = normwise_rel(y[off:off + rows], want)
        say("fused qkv", S.TYPE_NAMES[gtype], name, "normwise", err)
        assert err <= 1e-4, (name, err)
        off += rows


@pytest.mark.parametrize("gtype,hidden,rows", ((S.Q4_K, 2048, 5120), (S.Q5_K, 2048, 5120),
                                               (S.Q6_K, 2048, 5120), (S.Q8_0, 2048, 5120),
                                               (S.Q4_K, 4096, 2048)))
def test_fused_norm_projection(hip, port, gtype, hidden, rows):
    """The q/k/v projection with the residual add and attention RMSNorm in its
    staging: the updated residual bit for bit, the projection within 1e-4
    normwise of the oracle's tensor_linear of pko_add_rms_norm's row."""
    g = S.rng(400 + gtype + hidden)
    enc = S.quant_matrix(gtype, rows, hidden, g)
    h = S.normal_f32(g, hidden) * np.float32(4)
    d = S.normal_f32(g, hidden)
    nw = (1 + 0.125 * np.random.default_rng(hidden).random(hidden)).astype(np.float32)
    w = hip.upload(gtype, hidden, rows, enc)
    try:
        for delta in (d, None):
            gh, gy = hip.matvec_add_rmsnorm(w, h, delta, nw, 1e-6)
            ch, cn = port.add_rms_norm(h.reshape(1, -1), None if delta is None else delta.reshape(1, -1),
                                       nw, 1e-6)
            assert np.array_equal(gh.view(np.uint32), ch[0].view(np.uint32))
            err = normwise_rel(gy, port.linear(gtype, enc, hidden, rows, cn[0]))
            say("fused norm projection", S.TYPE_NAMES[gtype], hidden, rows, "delta",
                delta is not None, "normwise", err)
            assert err <= 1e-4, err
    finally:
        w.release()


def test_fused_norm_projection_unsupported_width(hip):
    """Widths the one-launch kernel does not cover are refused, not run."""
    from pokitlms_amd.backend import Unsupported
    g = S.rng(77)
    hidden, rows = 8192, 64
    w = hip.upload(S.Q4_K, hidden, rows, S.quant_matrix(S.Q4_K, rows, hidden, g))
    try:
        x = S.normal_f32(g, hidden)
        with pytest.raises(Unsupported):
            hip.matvec_add_rmsnorm(w, x, None, np.ones(hidden, np.float32), 1e-6)
    finally:
        w.release()


ATTN = (  # heads, kv_heads, head_dim, capacity, steps
    (32, 4, 128, 512, 48),   # config 5
    (32, 4, 128, 16, 40),    # the ring wraps
    (8, 2, 64, 12, 20),
    (4, 1, 256, 32, 8),
)


def _attn_inputs(seed, heads, kv_heads, head_dim, steps):
    g = np.random.default_rng(seed)
    q = g.standard_normal((steps, heads * head_dim)).astype(np.float32)
    k = (g.standard_normal((steps, kv_heads * head_dim)) * 3).astype(np.float32)
    v = g.standard_normal((steps, kv_heads * head_dim)).astype(np.float32)
    qn = (1 + 0.5 * g.random(head_dim)).astype(np.float32)
    kn = (1 + 0.5 * g.random(head_dim)).astype(np.float32)
    return qn, kn, q, k, v


@pytest.mark.parametrize("case", ATTN)
def test_attention_fast_and_reference_order(hip, port, case):
    from pokitlms_amd.model import libm_expf_pairs
    heads, kv_heads, head_dim, capacity, steps = case
    args = _attn_inputs(sum(case), heads, kv_heads, head_dim, steps)
    want = port.attention_steps(heads, kv_heads, head_dim, capacity, 1e-6, 1e6, *args)
    fast = hip.attention_steps(heads, kv_heads, head_dim, capacity, 1e-6, 1e6, *args)
    errs = [normwise_rel(fast[t], want[t]) for t in range(steps)]
    say("attention", case, "fast: worst normwise", max(errs), "at position", int(np.argmax(errs)))
    assert max(errs) <= 1e-4
    ref = hip.attention_steps(heads, kv_heads, head_dim, capacity, 1e-6, 1e6, *args,
                              reference_order=True, libm_expf_pairs=libm_expf_pairs())
    same = np.sum(ref.view(np.uint32) == want.view(np.uint32))
    say("attention", case, "reference order: bit-equal", int(same), "of", want.size)
    assert np.array_equal(ref.view(np.uint32), want.view(np.uint32))
