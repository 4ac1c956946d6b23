"""GPU parity of the batched MoE prefill (pk_hip_moe_prefill) through the C ABI.

The reference prefills one token at a time through the MoE block
(src/qwen3_moe_runner.cpp:785-790, block at :643-692), so every token of a
batch must get the routes and output of a single-token pass: ids and route
order bit-exact against the CPU oracle, route weights equal to the decode
path's bit for bit (same arithmetic), outputs within normwise relative error
1e-4 of the CPU's (the expert GEMMs run on FP32 MFMA in another order).
"""
import numpy as np
import pytest

from pokitlms_amd import synth as S
from tests.conftest import normwise_rel
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu

QUANT = (S.Q4_0, S.Q4_1, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K)
TOL = 1e-4


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def say(*a):
    print(*a, flush=True)


def check_against_cpu(blk, x, y, ids, probs, tokens):
    worst = 0.0
    for t in tokens:
        cy, cids, cprobs = blk.forward(x[t])
        assert np.array_equal(ids[t], cids), (t, ids[t], cids)
        assert np.max(np.abs(probs[t] - cprobs)) <= TOL * np.max(cprobs), t
        worst = max(worst, normwise_rel(y[t], cy))
    assert worst <= TOL, worst
    return worst


def check_against_decode(hip, h, x, y, ids, probs, tokens):
    worst = 0.0
    for t in tokens:
        dy, dids, dprobs = hip.moe_decode(h, x[t])
        assert np.array_equal(ids[t], dids), (t, ids[t], dids)
        assert np.array_equal(bits(probs[t]), bits(dprobs)), t
        worst = max(worst, normwise_rel(y[t], dy))
    assert worst <= TOL, worst
    return worst


# (hidden, experts, ffn, top_k, gate/up type, down type, tokens)
SHAPES = (
    (512, 16, 256, 2, S.Q4_K, S.Q6_K, 1),
    (512, 16, 256, 4, S.Q4_K, S.Q6_K, 37),
    (512, 32, 256, 8, S.Q5_K, S.Q8_0, 100),
    (1024, 64, 512, 8, S.Q4_K, S.Q6_K, 65),
    (2048, 64, 768, 6, S.Q6_K, S.Q4_K, 33),
    (3072, 32, 1024, 4, S.Q4_0, S.Q5_K, 20),
    (4096, 64, 1536, 8, S.Q4_K, S.Q6_K, 24),
)


@pytest.mark.parametrize("shape", SHAPES,
                         ids=lambda s: f"{s[0]}x{s[1]}x{s[2]}k{s[3]}t{s[4]}-{s[5]}n{s[6]}")
def test_prefill_shapes_against_cpu(hip, port, shape):
    hidden, experts, ffn, k, gt, dt, tokens = shape
    say("prefill shape", shape)
    layer = S.moe_layer(seed=210 + hidden + ffn + tokens, hidden=hidden, experts=experts,
                        ffn=ffn, gate_type=gt, up_type=gt, down_type=dt, top_k=k)
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(S.rng(2100 + tokens), tokens * hidden).reshape(tokens, hidden)
    y, ids, probs = hip.moe_prefill(h, x)
    assert y.shape == (tokens, hidden) and ids.shape == (tokens, k)
    worst = check_against_cpu(port.moe(layer), x, y, ids, probs, range(tokens))
    check_against_decode(hip, h, x, y, ids, probs, range(tokens))
    say("  worst normwise vs cpu", worst)
    h.release()


@pytest.mark.parametrize("gt", QUANT)
def test_prefill_every_type_pair(hip, port, gt):
    """Each gate/up type with each down type (the dequantisation into the MFMA
    tiles is written per format)."""
    for dt in QUANT:
        say("prefill types", S.TYPE_NAMES[gt], S.TYPE_NAMES[dt])
        layer = S.moe_layer(seed=300 + gt * 16 + dt, hidden=512, experts=16, ffn=256,
                            gate_type=gt, up_type=gt, down_type=dt, top_k=4)
        h = hip.upload_moe_layer(layer)
        x = S.normal_f32(S.rng(3000 + dt), 40 * 512).reshape(40, 512)
        y, ids, probs = hip.moe_prefill(h, x)
        check_against_cpu(port.moe(layer), x, y, ids, probs, range(40))
        h.release()


@pytest.fixture(scope="module")
def c4(hip):
    """The C3 layer (2048 -> 768, 128 experts, top-8, Q4_K gate/up, Q6_K down)
    with a router that realises a Zipf(1.1) expert load over 512 tokens."""
    layer = G.c3_layer()
    layer.router, _ = S.zipf_router(layer.experts, layer.hidden, layer.top_k, seed=404)
    x = S.zipf_tokens(404, 512, layer.hidden)
    h = hip.upload_moe_layer(layer)
    yield layer, h, x
    h.release()


def test_prefill_c4_zipf(hip, port, c4):
    layer, h, x = c4
    hip.reset_stats()
    y, ids, probs = hip.moe_prefill(h, x)
    st = hip.stats()
    assert st["prefill_calls"] == 1 and st["prefill_tokens"] == 512
    counts = np.bincount(ids.ravel().astype(np.int64), minlength=layer.experts)
    fit = S.zipf_fit(counts)
    say("c4 load: max", counts.max(), "touched", int((counts > 0).sum()), "fit", fit)
    assert counts.max() >= 450 and 0.8 <= fit <= 1.5
    dec = check_against_decode(hip, h, x, y, ids, probs, range(512))
    cpu = check_against_cpu(port.moe(layer), x, y, ids, probs, range(0, 512, 8))
    say("c4 worst normwise: vs decode", dec, "vs cpu", cpu)


def test_prefill_deterministic(hip, c4):
    _, h, x = c4
    y0, i0, p0 = hip.moe_prefill(h, x[:200])
    for _ in range(2):
        y1, i1, p1 = hip.moe_prefill(h, x[:200])
        assert np.array_equal(bits(y0), bits(y1)) and np.array_equal(i0, i1)
        assert np.array_equal(bits(p0), bits(p1))


def test_prefill_one_hot_expert_groups(hip, port):
    """An all-zero router ties every logit, so every token takes experts
    0..k-1: each group holds all 4096 tokens (128 full tiles per expert)."""
    layer = S.moe_layer(seed=410, hidden=512, experts=8, ffn=256, top_k=2)
    layer.router = np.zeros((8, 512), np.float32)
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(S.rng(411), 4096 * 512).reshape(4096, 512)
    y, ids, probs = hip.moe_prefill(h, x)
    assert np.array_equal(ids, np.tile(np.arange(2, dtype=np.uint32), (4096, 1)))
    check_against_cpu(port.moe(layer), x, y, ids, probs, range(0, 4096, 97))
    check_against_decode(hip, h, x, y, ids, probs, range(0, 4096, 31))
    h.release()


def test_prefill_max_tokens_random_routes(hip, port):
    layer = S.moe_layer(seed=420, hidden=512, experts=32, ffn=256, top_k=8)
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(S.rng(421), 4096 * 512).reshape(4096, 512)
    y, ids, probs = hip.moe_prefill(h, x)
    check_against_decode(hip, h, x, y, ids, probs, range(4096))
    check_against_cpu(port.moe(layer), x, y, ids, probs, range(0, 4096, 61))
    h.release()


def test_prefill_near_ties_take_the_exact_path(hip, port):
    g = S.rng(430)
    router = S.normal_f32(g, 32 * 512, 0.02).reshape(32, 512)
    for j in range(0, 32, 2):
        router[j + 1] = router[j]
        kk = int(g.integers(0, 512))
        router[j + 1, kk] = np.nextafter(router[j, kk], np.float32(1))
    layer = S.moe_layer(seed=431, hidden=512, experts=32, ffn=256, top_k=8)
    layer.router = router
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(g, 48 * 512).reshape(48, 512)
    hip.reset_stats()
    y, ids, probs = hip.moe_prefill(h, x)
    st = hip.stats()
    say("prefill near-tie fallbacks", st["router_fallbacks"])
    assert st["router_fallbacks"] > 0
    check_against_cpu(port.moe(layer), x, y, ids, probs, range(48))
    h.release()


def test_prefill_non_finite_token_is_a_runtime_error(hip, port):
    from pokitlms_amd.backend import HipError
    layer = S.moe_layer(seed=440, hidden=512, experts=16, ffn=256, top_k=4)
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(S.rng(441), 20 * 512).reshape(20, 512)
    bad = x.copy()
    bad[3, 17] = np.nan
    with pytest.raises(HipError) as ex:
        hip.moe_prefill(h, bad)
    assert ex.value.status == 2 and "non-finite" in str(ex.value)
    # the next batch starts from clean counts and matches the CPU
    y, ids, probs = hip.moe_prefill(h, x)
    check_against_cpu(port.moe(layer), x, y, ids, probs, range(20))
    h.release()


def test_prefill_unsupported_shapes(hip):
    from pokitlms_amd.backend import Unsupported
    layer = S.moe_layer(seed=450, hidden=512, experts=16, ffn=256, gate_type=S.Q4_K,
                        up_type=S.Q5_K, down_type=S.Q6_K, top_k=4)
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(S.rng(451), 4 * 512).reshape(4, 512)
    with pytest.raises(Unsupported):
        hip.moe_prefill(h, x)  # gate and up must share a format
    h.release()
    h = hip.upload_moe_layer(S.moe_layer(seed=452, hidden=512, experts=16, ffn=256, top_k=4))
    with pytest.raises(ValueError, match="token count"):
        hip.moe_prefill(h, np.zeros((0, 512), np.float32))
    with pytest.raises(ValueError, match="token count"):
        hip.moe_prefill(h, np.zeros((4097, 512), np.float32))
    h.release()


def test_prefill_graph_replays_match_eager(hip, c4):
    """After one eager call (which sizes the scratch), a captured prefill
    replays to the eager results each time, with eager work between."""
    import torch
    _, h, x = c4
    dev = torch.device("cuda:0")
    T = 96
    dx = torch.from_numpy(np.ascontiguousarray(x[:T])).to(dev)
    dy = torch.empty(T, 2048, device=dev)
    di = torch.empty(T, 8, dtype=torch.int32, device=dev)
    dp = torch.empty(T, 8, device=dev)
    stream = torch.cuda.Stream()

    def run(s):
        hip.moe_prefill_async(h, dx.data_ptr(), T, dy.data_ptr(), di.data_ptr(), dp.data_ptr(), s)
    with torch.cuda.stream(stream):
        run(stream.cuda_stream)
    hip.sync(stream.cuda_stream)
    y_ref, i_ref, p_ref = dy.clone(), di.clone(), dp.clone()
    y_sync, ids_sync, _ = hip.moe_prefill(h, x[:T])
    assert np.array_equal(bits(y_ref.cpu().numpy()), bits(y_sync))
    assert np.array_equal(i_ref.cpu().numpy().astype(np.uint32), ids_sync)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        dy.zero_()
        di.zero_()
        dp.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        hip.sync(0)
        assert torch.equal(dy, y_ref) and torch.equal(di, i_ref) and torch.equal(dp, p_ref), rep
        hip.moe_decode(h, x[rep])  # eager work between replays


def test_capture_refuses_scratch_growth_and_old_graphs_survive_it():
    """A fresh context: a call under stream capture that would need more
    scratch than earlier calls sized is refused with INVALID_ARGUMENT (an
    allocation cannot be part of the graph); an eager call may grow it, and
    a graph captured before the growth still replays to its eager results,
    because the old scratch is kept until the context is destroyed."""
    import torch
    from pokitlms_amd.backend import HipBackend
    layer = S.moe_layer(seed=777, hidden=512, experts=16, ffn=256, top_k=4)
    x = S.normal_f32(S.rng(778), 64 * 512).reshape(64, 512)
    dev = torch.device("cuda:0")
    with HipBackend(0) as fresh:
        h = fresh.upload_moe_layer(layer)
        dx = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        dy = torch.empty(64, 512, device=dev)
        di = torch.empty(64, 4, dtype=torch.int32, device=dev)
        dp = torch.empty(64, 4, device=dev)
        stream = torch.cuda.Stream()

        def run(s, tokens):
            fresh.moe_prefill_async(h, dx.data_ptr(), tokens, dy.data_ptr(), di.data_ptr(),
                                    dp.data_ptr(), s)
        with torch.cuda.stream(stream):
            run(stream.cuda_stream, 8)
        fresh.sync(stream.cuda_stream)
        y8, i8, p8 = dy[:8].clone(), di[:8].clone(), dp[:8].clone()
        g8 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g8, stream=stream):
            run(torch.cuda.current_stream().cuda_stream, 8)
        refused = None
        g64 = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g64, stream=stream):
                run(torch.cuda.current_stream().cuda_stream, 64)
        except ValueError as e:  # INVALID_ARGUMENT
            refused = e
        assert refused is not None and "outside stream capture" in str(refused), refused
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):  # eager: grows the scratch
            run(stream.cuda_stream, 64)
        fresh.sync(stream.cuda_stream)
        y64, i64 = dy.clone(), di.clone()
        assert torch.equal(i64[:8], i8)
        assert normwise_rel(y64[:8].cpu().numpy(), y8.cpu().numpy()) <= TOL
        for rep in range(3):
            dy.zero_()
            di.zero_()
            dp.zero_()
            torch.cuda.synchronize()
            g8.replay()
            torch.cuda.synchronize()
            fresh.sync(0)
            assert torch.equal(dy[:8], y8) and torch.equal(di[:8], i8), rep
            assert torch.equal(dp[:8], p8), rep
            fresh.moe_decode(h, x[rep])  # eager work between replays
        del g8, g64
        h.release()


def test_prefill_kernel_timing(hip, c4):
    _, h, x = c4
    hip.set_kernel_timing(True)
    try:
        hip.reset_stats()
        hip.moe_prefill(h, x)
        st = hip.stats()
        say("prefill 512 tokens:", st["prefill_ns"] / 1e3, "us")
        assert st["prefill_ns"] > 0
    finally:
        hip.set_kernel_timing(False)
