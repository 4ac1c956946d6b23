"""Qwen3.5-MoE block (src/qwen35_runner.cpp:131-173 select_experts, :670-764
the MoE block with its shared expert).

CPU: the C restatement (oracle/pk_oracle.c) against the reference's own
vectors (tests/golden/qwen35_golden.npz, written by make_qwen35_golden.py
from the compiled reference), bit for bit, and against the routing
invariants.  GPU: pk_hip_moe35_decode against the same vectors -- ids
bit-exact, weights and outputs within 1e-4 normwise (FP32 reassociation of
the softmax denominator and of the dot products)."""
import os

import numpy as np
import pytest

import oracle
from pokitlms_amd import synth as S
from tests.conftest import normwise_rel
from tests.golden.make_golden import route_cases
from tests.golden.make_qwen35_golden import LAYERS, layer_tokens

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qwen35_golden.npz")


@pytest.fixture(scope="module")
def g35():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def port():
    if not oracle.available("port"):
        oracle.build(reference=False)
    return oracle.Oracle("port")


def test_golden_select_experts(port, g35):
    for i, (lg, k, norm) in enumerate(route_cases()):
        ids, w = port.select_experts(lg, k, norm)
        assert np.array_equal(ids, g35[f"select{i}_ids"]), i
        assert np.array_equal(w.view(np.uint32), g35[f"select{i}_weights"].view(np.uint32)), i


def test_select_experts_invariants(port):
    """Order by brute-force lexsort (logit desc, id asc); weights the FP32
    softmax of the selected logits (to an ulp-scale tolerance: numpy's exp is
    not the C library's); renormalised weights sum to one."""
    g = S.rng(77)
    for trial in range(40):
        n = int(g.integers(2, 200))
        k = int(g.integers(1, min(n, 16) + 1))
        lg = S.normal_f32(g, n, 2.0)
        if trial % 4 == 0:
            lg[g.integers(0, n, 3)] = lg[0]  # ties
        ids, w = port.select_experts(lg, k, False)
        order = np.lexsort((np.arange(n), -lg.astype(np.float64)))[:k]
        assert np.array_equal(ids, order)
        e = np.exp(lg.astype(np.float64) - lg.max())
        assert np.allclose(w, (e / e.sum())[ids], rtol=1e-5, atol=0)
        _, wn = port.select_experts(lg, k, True)
        assert abs(float(np.sum(wn, dtype=np.float64)) - 1.0) < 1e-5
    with pytest.raises(oracle.OracleError):
        port.select_experts(np.array([0.0, np.inf], np.float32), 1, True)


@pytest.mark.parametrize("name,kw,n", LAYERS, ids=[l[0] for l in LAYERS])
def test_golden_moe35_block(port, g35, name, kw, n):
    layer, xs = layer_tokens(name, kw, n)
    assert S.digest(layer.router, layer.gate, layer.up, layer.down, layer.shared_router,
                    layer.shared_gate, layer.shared_up, layer.shared_down, xs) == str(g35[f"{name}_digest"])
    blk = port.moe35(layer)
    ys = []
    for t, x in enumerate(xs):
        y, ids, w = blk.forward(x)
        assert np.array_equal(ids, g35[f"{name}_ids"][t])
        assert np.array_equal(w.view(np.uint32), g35[f"{name}_weights"][t].view(np.uint32))
        ys.append(y)
    ys = np.stack(ys)
    assert np.array_equal(ys[:4].view(np.uint32), g35[f"{name}_y"].view(np.uint32))
    assert S.digest(ys) == str(g35[f"{name}_ysum"])


def test_moe35_block_from_its_parts(port):
    """The block equals routed experts weighted by (weight * scale) plus the
    shared expert weighted by the sigmoid of its gate, composed here from the
    oracle's own linear and select_experts."""
    layer, xs = layer_tokens(*LAYERS[1][:2], 2)
    L = layer
    x = xs[0]
    logits = port.linear(S.F32, L.router.view(np.uint8), L.hidden, L.experts, x)
    ids, w = port.select_experts(logits, L.top_k, L.normalize)

    def ffn(gt, g, ut, u, dt, d, width):
        gv = port.linear(gt, g, L.hidden, width, x).astype(np.float64)
        uv = port.linear(ut, u, L.hidden, width, x).astype(np.float64)
        act = (gv / (1.0 + np.exp(-gv)) * uv).astype(np.float32)
        return port.linear(dt, d, width, L.hidden, act).astype(np.float64)

    want = np.zeros(L.hidden)
    for r, e in enumerate(ids):
        want += float(w[r]) * L.scale * ffn(L.gate_type, L.gate[e], L.up_type, L.up[e], L.down_type,
                                            L.down[e], L.ffn)
    gate_value = float(port.linear(S.F32, L.shared_router.view(np.uint8), L.hidden, 1, x)[0])
    want += 1.0 / (1.0 + np.exp(-gate_value)) * ffn(L.gate_type, L.shared_gate, L.up_type,
                                                      L.shared_up, L.down_type, L.shared_down,
                                                      L.shared_ffn)
    y, ids2, _ = port.moe35(L).forward(x)
    assert np.array_equal(ids, ids2)
    assert normwise_rel(y, want) < 1e-5


# ---- GPU ------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,n", LAYERS, ids=[l[0] for l in LAYERS])
def test_gpu_moe35_decode_golden(hip, g35, name, kw, n):
    layer, xs = layer_tokens(name, kw, n)
    h = hip.upload_moe35_layer(layer)
    worst_y = worst_w = 0.0
    try:
        for t, x in enumerate(xs):
            y, ids, w = hip.moe35_decode(h, x)
            assert np.array_equal(ids, g35[f"{name}_ids"][t]), (t, ids, g35[f"{name}_ids"][t])
            worst_w = max(worst_w, normwise_rel(w, g35[f"{name}_weights"][t] * np.float32(kw["scale"])))
            if t < 4:
                worst_y = max(worst_y, normwise_rel(y, g35[f"{name}_y"][t]))
    finally:
        h.release()
    print(f"qwen35 {name}: weights normwise {worst_w:.2e}, outputs {worst_y:.2e}", flush=True)
    assert worst_w <= 1e-4 and worst_y <= 1e-4


@pytest.mark.gpu
def test_gpu_moe35_async_and_errors(hip, port):
    import ctypes
    import torch
    from pokitlms_amd.backend import HipError, Unsupported
    layer, xs = layer_tokens(*LAYERS[1][:2], 3)
    h = hip.upload_moe35_layer(layer)
    try:
        dev = torch.device("cuda:0")
        X = torch.from_numpy(xs[2].copy()).to(dev)
        Y = torch.empty(layer.hidden, device=dev)
        I = torch.empty(layer.top_k, dtype=torch.int32, device=dev)
        W = torch.empty(layer.top_k, device=dev)
        torch.cuda.synchronize()
        hip.moe35_decode_async(h, X.data_ptr(), Y.data_ptr(), I.data_ptr(), W.data_ptr())
        hip.sync()
        y, ids, w = hip.moe35_decode(h, xs[2])
        assert np.array_equal(Y.cpu().numpy().view(np.uint32), y.view(np.uint32))
        assert np.array_equal(I.cpu().numpy().astype(np.uint32), ids)
        # a shared expert of another width is not covered by the fused kernels
        narrow = hip.upload(layer.gate_type, layer.hidden, 256,
                            S.quant_matrix(layer.gate_type, 256, layer.hidden, S.rng(1)))
        from pokitlms_amd.backend import Moe35LayerHandles
        bad = Moe35LayerHandles(h, h.shared[0], narrow, h.shared[2], h.shared[3])
        with pytest.raises((Unsupported, ValueError)):
            hip.moe35_decode(bad, xs[0])
        narrow.release()
        # non-finite router logits: route_experts' error
        poison = xs[0].copy()
        poison[3] = np.inf
        with pytest.raises(HipError):
            hip.moe35_decode(h, poison)
    finally:
        h.release()


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,n", LAYERS, ids=[l[0] for l in LAYERS])
def test_gpu_moe35_prefill_matches_decode_and_golden(hip, g35, name, kw, n):
    """The batched Qwen3.5 block (pk_hip_moe35_prefill): per token the decode
    path's ids and weights bit for bit (the same router sums, bounds and
    weight code), outputs within 1e-4 normwise of the decode path and of the
    reference's golden outputs."""
    layer, xs = layer_tokens(name, kw, n)
    extra = S.normal_f32(S.rng(4040), 61 * layer.hidden).reshape(61, layer.hidden)
    X = np.concatenate([xs, extra])
    h = hip.upload_moe35_layer(layer)
    worst = 0.0
    try:
        y, ids, w = hip.moe35_prefill(h, X)
        for t in range(X.shape[0]):
            dy, dids, dw = hip.moe35_decode(h, X[t])
            assert np.array_equal(ids[t], dids), (t, ids[t], dids)
            assert np.array_equal(w[t].view(np.uint32), dw.view(np.uint32)), t
            worst = max(worst, normwise_rel(y[t], dy))
        for t in range(len(xs)):
            assert np.array_equal(ids[t], g35[f"{name}_ids"][t]), t
        for t in range(min(4, len(xs))):
            assert normwise_rel(y[t], g35[f"{name}_y"][t]) <= 1e-4, t
    finally:
        h.release()
    print(f"qwen35 prefill {name}: {X.shape[0]} tokens, worst normwise vs decode {worst:.2e}",
          flush=True)
    assert worst <= 1e-4


@pytest.mark.gpu
def test_gpu_moe35_prefill_shared_expert_matters(hip):
    """The shared expert's share is in the batched output: with its gate row
    scaled so sigmoid saturates near 0 or 1 the outputs move by the shared
    expert's output (both paths agree either way)."""
    layer, xs = layer_tokens(*LAYERS[1][:2], 16)
    outs = []
    for gain in (-50.0, 50.0):
        layer.shared_router = (np.sign(xs[0]) * np.float32(gain / layer.hidden)).astype(np.float32)
        h = hip.upload_moe35_layer(layer)
        try:
            y, _, _ = hip.moe35_prefill(h, xs[:1])
            dy, _, _ = hip.moe35_decode(h, xs[0])
            assert normwise_rel(y[0], dy) <= 1e-4
            outs.append(y[0])
        finally:
            h.release()
    assert normwise_rel(outs[0], outs[1]) > 1e-2


@pytest.mark.gpu
def test_gpu_moe35_prefill_async_graph_and_errors(hip):
    """pk_hip_moe35_prefill_async on device buffers equals the synchronous
    call bit for bit, also when captured in a HIP graph and replayed; a
    narrower shared expert and a non-finite token are rejected like the
    decode path rejects them."""
    import torch
    from pokitlms_amd.backend import HipError, Moe35LayerHandles, Unsupported
    layer, xs = layer_tokens(*LAYERS[1][:2], 40)
    h = hip.upload_moe35_layer(layer)
    try:
        y, ids, w = hip.moe35_prefill(h, xs)
        dev = torch.device("cuda:0")
        X = torch.from_numpy(xs.copy()).to(dev)
        Y = torch.empty(xs.shape, device=dev)
        I = torch.empty((xs.shape[0], layer.top_k), dtype=torch.int32, device=dev)
        W = torch.empty((xs.shape[0], layer.top_k), device=dev)
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            hip.moe35_prefill_async(h, X.data_ptr(), xs.shape[0], Y.data_ptr(), I.data_ptr(),
                                    W.data_ptr(), s.cuda_stream)
        s.synchronize()
        assert np.array_equal(Y.cpu().numpy().view(np.uint32), y.view(np.uint32))
        assert np.array_equal(I.cpu().numpy().astype(np.uint32), ids)
        assert np.array_equal(W.cpu().numpy().view(np.uint32), w.view(np.uint32))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            hip.moe35_prefill_async(h, X.data_ptr(), xs.shape[0], Y.data_ptr(), I.data_ptr(),
                                    W.data_ptr(), torch.cuda.current_stream().cuda_stream)
        for _ in range(3):
            Y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(Y.cpu().numpy().view(np.uint32), y.view(np.uint32))
        narrow = hip.upload(layer.gate_type, layer.hidden, 256,
                            S.quant_matrix(layer.gate_type, 256, layer.hidden, S.rng(1)))
        bad = Moe35LayerHandles(h, h.shared[0], narrow, h.shared[2], h.shared[3])
        with pytest.raises((Unsupported, ValueError)):
            hip.moe35_prefill(bad, xs[:4])
        narrow.release()
        poison = xs[:4].copy()
        poison[2, 5] = np.nan
        with pytest.raises(HipError):
            hip.moe35_prefill(h, poison)
    finally:
        h.release()
