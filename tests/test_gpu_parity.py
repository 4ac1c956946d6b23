"""GPU parity: libpokit_hip.so (through its C ABI) against the CPU oracle.

Bars: expert ids and routing order bit-exact; FP32
outputs within normwise relative error max|gpu-cpu| / max|cpu| <= 1e-4; on
dyadic-exact inputs every output bit-exact.  The reference's own Vulkan
harness tolerance |cpu-gpu| <= 1e-3 + 2e-5|cpu| (tests/vulkan_linear_cases.hpp:81)
is checked as well on its 37 x 512 shapes.
"""
import numpy as np
import pytest

from pokitlms_amd import synth as S
from pokitlms_amd.backend import HipError
from tests.conftest import normwise_rel
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu

QUANT = (S.Q4_0, S.Q4_1, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K)
# the other formats tensor_linear dispatches (src/tensor_linear.cpp:176-187)
QUANT_MORE = (S.Q5_0, S.Q5_1, S.Q2_K, S.Q3_K)
FLOAT = (S.F32, S.F16, S.BF16)
TOL = 1e-4


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def say(*a):
    print(*a, flush=True)


# ---- matvec -------------------------------------------------------------------------

@pytest.mark.parametrize("gtype", FLOAT + QUANT + QUANT_MORE)
def test_reference_harness_shapes(hip, port, gtype):
    """37 rows x 512 (257 for floats) of xorshift-style random bytes with the
    harness's fixed scales, three rounds with x *= -0.75
    (tests/vulkan_linear_cases.hpp:31-88)."""
    say("harness", S.TYPE_NAMES[gtype])
    w, x, inn = G.small_inputs(gtype, seed=123)
    if gtype in QUANT:
        blocks = w.reshape(-1, S.BLOCK_BYTES[gtype])
        for off in S.SCALE_OFFSETS[gtype]:
            val = 0x2800 if off in (0, 208) else 0x2400
            blocks[:, off] = val & 0xFF
            blocks[:, off + 1] = val >> 8
    wt = hip.upload(gtype, inn, 37, w)
    for _ in range(3):
        cpu = port.linear(gtype, w, inn, 37, x)
        gpu = hip.matvec(wt, x)
        assert np.all(np.isfinite(gpu))
        assert np.all(np.abs(cpu - gpu) <= 1e-3 + 2e-5 * np.abs(cpu))
        assert normwise_rel(gpu, cpu) <= TOL
        x = (x * np.float32(-0.75)).astype(np.float32)
    wt.release()


@pytest.mark.parametrize("gtype", QUANT + QUANT_MORE)
@pytest.mark.parametrize("batch", (1, 2, 4, 8))
def test_dyadic_bit_exact(hip, port, gtype, batch):
    say("dyadic", S.TYPE_NAMES[gtype], batch)
    g = S.rng(500 + gtype * 10 + batch)
    rows, inn = 96, 2048
    w = S.dyadic_matrix(gtype, rows, inn, g)
    xs = np.stack([S.dyadic_vector(g, inn) for _ in range(batch)])
    wt = hip.upload(gtype, inn, rows, w)
    gpu = hip.matvec(wt, xs)
    for b in range(batch):
        cpu = port.linear(gtype, w, inn, rows, xs[b])
        assert np.array_equal(bits(gpu[b]), bits(cpu)), (S.TYPE_NAMES[gtype], batch, b)
    wt.release()


def test_c1_q4k_4096(hip, golden):
    say("c1")
    w, x = G.c1_inputs()
    wt = hip.upload(S.Q4_K, 4096, 4096, w)
    gpu = hip.matvec(wt, x)
    err = normwise_rel(gpu, golden["c1_y"])
    say("c1 normwise", err)
    assert err <= TOL
    wt.release()


@pytest.mark.parametrize("gtype", QUANT)
@pytest.mark.parametrize("shape", G.C2_SHAPES)
def test_c2_sweep(hip, port, golden, gtype, shape):
    rows, inn = shape
    say("c2", S.TYPE_NAMES[gtype], rows, inn)
    w, xs = G.c2_inputs(gtype, rows, inn)
    key = f"c2_{S.TYPE_NAMES[gtype]}_{rows}x{inn}"
    wt = hip.upload(gtype, inn, rows, w)
    cpu = np.stack([port.linear(gtype, w, inn, rows, xs[b]) for b in range(8)])
    assert np.array_equal(bits(cpu[0]), bits(golden[key + "_y0"]))
    for batch in (1, 4, 8):
        gpu = hip.matvec(wt, xs[:batch])
        for b in range(batch):
            err = normwise_rel(gpu[b], cpu[b])
            assert err <= TOL, (batch, b, err)
    wt.release()


@pytest.mark.parametrize("gtype", QUANT)
@pytest.mark.parametrize("shape", G.C2_SHAPES)
def test_reference_order_matvec_bit_exact(hip, golden, gtype, shape):
    """pk_hip_matvec_reference_order returns the reference's bits (the golden
    vectors come from the compiled reference itself)."""
    rows, inn = shape
    w, xs = G.c2_inputs(gtype, rows, inn)
    key = f"c2_{S.TYPE_NAMES[gtype]}_{rows}x{inn}"
    wt = hip.upload(gtype, inn, rows, w)
    y = hip.matvec_reference_order(wt, xs[0])
    same = int(np.sum(bits(y) == bits(golden[key + "_y0"])))
    say("reference order", S.TYPE_NAMES[gtype], shape, "bit-equal", same, "of", rows)
    assert same == rows
    wt.release()


@pytest.mark.parametrize("gtype", QUANT_MORE)
def test_more_formats_against_the_reference(hip, port, golden, gtype):
    """Q5_0, Q5_1, Q2_K and Q3_K on the reference harness shape: the fast
    matvec within 1e-4 normwise of the compiled reference's vector, the
    reference-order matvec equal to it bit for bit, and random 2048-wide rows
    at batch 1/3/8 within 1e-4 of the oracle."""
    w, x, inn = G.small_inputs(gtype)
    key = f"small_{S.TYPE_NAMES[gtype]}"
    wt = hip.upload(gtype, inn, 37, w)
    assert normwise_rel(hip.matvec(wt, x), golden[key + "_y"]) <= TOL
    assert np.array_equal(bits(hip.matvec_reference_order(wt, x)), bits(golden[key + "_y"]))
    wt.release()
    g = S.rng(80 + gtype)
    w = S.quant_matrix(gtype, 300, 2048, g)
    xs = np.stack([S.normal_f32(g, 2048) for _ in range(8)])
    wt = hip.upload(gtype, 2048, 300, w)
    for batch in (1, 3, 8):
        gpu = hip.matvec(wt, xs[:batch])
        for b in range(batch):
            assert normwise_rel(gpu[b], port.linear(gtype, w, 2048, 300, xs[b])) <= TOL, (batch, b)
    wt.release()


def test_reference_order_router_and_c1(hip, port, golden):
    w, x = G.c1_inputs()
    wt = hip.upload(S.Q4_K, 4096, 4096, w)
    assert np.array_equal(bits(hip.matvec_reference_order(wt, x)), bits(golden["c1_y"]))
    wt.release()
    g = S.rng(71)
    router = S.normal_f32(g, 128 * 2048, 0.02).reshape(128, 2048)
    xr = S.normal_f32(g, 2048)
    rt = hip.upload(S.F32, 2048, 128, router)
    cpu = port.linear(S.F32, router.view(np.uint8), 2048, 128, xr)
    assert np.array_equal(bits(hip.matvec_reference_order(rt, xr)), bits(cpu))
    rt.release()


@pytest.mark.parametrize("batch", (2, 3, 5, 6, 7))
def test_odd_batches(hip, port, batch):
    g = S.rng(40 + batch)
    w = S.quant_matrix(S.Q6_K, 300, 1536, g)
    xs = S.normal_f32(g, batch * 1536).reshape(batch, 1536)
    wt = hip.upload(S.Q6_K, 1536, 300, w)
    gpu = hip.matvec(wt, xs)
    for b in range(batch):
        assert normwise_rel(gpu[b], port.linear(S.Q6_K, w, 1536, 300, xs[b])) <= TOL
    wt.release()


@pytest.mark.parametrize("gtype", QUANT + (S.Q2_K, S.Q3_K))
def test_staged_single_vector_widths(hip, port, gtype):
    """One vector through the kernel that stages x in LDS for the workgroup:
    widths whose last unit slot is partly absent (2304, 5120), two K-slices
    (5120, 8192), and a row count that makes each workgroup walk its loop
    more than once with a partial last pass (10,001 rows of 2048)."""
    g = S.rng(91 + gtype)
    for rows, inn in ((1000, 2304), (777, 4096), (1000, 5120), (513, 8192), (10001, 2048)):
        if inn % (256 if gtype in (S.Q4_K, S.Q5_K, S.Q6_K, S.Q2_K, S.Q3_K) else 32):
            continue
        w = S.quant_matrix(gtype, rows, inn, g)
        x = S.normal_f32(g, inn).reshape(1, inn)
        wt = hip.upload(gtype, inn, rows, w)
        gpu = hip.matvec(wt, x)[0]
        cpu = port.linear(gtype, w, inn, rows, x[0])
        err = normwise_rel(gpu, cpu)
        say("staged matvec", gtype, rows, inn, "normwise", err)
        assert err <= TOL, (rows, inn)
        wt.release()


@pytest.mark.parametrize("gtype", QUANT)
def test_staged_batched_widths(hip, port, gtype):
    """Two to four vectors through the staging kernel (each vector's pieces
    after the previous one's in LDS): one K-slice (1024 wide), two (2048,
    with 10,001 rows so workgroups loop with a partial last pass), and a width
    whose slices are narrower than a wave (1536), which takes the plain
    kernel; every vector checked against the CPU's linear."""
    g = S.rng(171 + gtype)
    for rows, inn in ((1000, 1024), (10001, 2048), (777, 1536)):
        w = S.quant_matrix(gtype, rows, inn, g)
        wt = hip.upload(gtype, inn, rows, w)
        for batch in (2, 3, 4):
            x = S.normal_f32(g, batch * inn).reshape(batch, inn)
            gpu = hip.matvec(wt, x)
            for b in range(batch):
                cpu = port.linear(gtype, w, inn, rows, x[b])
                err = normwise_rel(gpu[b], cpu)
                assert err <= TOL, (rows, inn, batch, b, err)
            say("staged batched matvec", gtype, rows, inn, batch, "ok")
        wt.release()


@pytest.mark.parametrize("gtype", (S.Q4_K, S.Q5_K, S.Q6_K, S.Q8_0, S.Q4_0))
def test_mfma_batched_widths(hip, port, gtype):
    """Five to eight vectors through the MFMA kernel: one 256-value range per
    wave with two row tiles (2048 wide), two and three ranges per wave with
    one tile (6144, 9216 wide: 12 waves), four (16384 wide, 16 waves; the
    K-quants), row counts that leave a partial tile; every vector against the
    CPU's linear."""
    g = S.rng(313 + gtype)
    shapes = [(1000, 2048), (777, 6144), (513, 9216)]
    if gtype in (S.Q4_K, S.Q5_K):
        shapes.append((300, 16384))
    for rows, inn in shapes:
        w = S.quant_matrix(gtype, rows, inn, g)
        wt = hip.upload(gtype, inn, rows, w)
        for batch in (5, 8):
            x = S.normal_f32(g, batch * inn).reshape(batch, inn)
            gpu = hip.matvec(wt, x)
            for b in range(batch):
                cpu = port.linear(gtype, w, inn, rows, x[b])
                err = normwise_rel(gpu[b], cpu)
                assert err <= TOL, (rows, inn, batch, b, err)
            say("mfma batched matvec", gtype, rows, inn, batch, "ok")
        wt.release()


@pytest.mark.parametrize("gtype", (S.Q4_K, S.Q5_K, S.Q6_K, S.Q8_0, S.Q4_0))
def test_mfma_k_sliced_shapes(hip, port, gtype):
    """The K-sliced MFMA kernel (grids of at most 128 row groups) with two,
    three and four 256-value ranges per workgroup (2000x4096, 2048x6144,
    2048x8192: 8, 8 and 8 K slices added in slice order by the reduce
    launch), a partial last row group, and 4, 5 and 8 vectors; every vector
    against the CPU's linear."""
    g = S.rng(911 + gtype)
    for rows, inn in ((2000, 4096), (2048, 6144), (2048, 8192)):
        w = S.quant_matrix(gtype, rows, inn, g)
        wt = hip.upload(gtype, inn, rows, w)
        for batch in (4, 5, 8):
            x = S.normal_f32(g, batch * inn).reshape(batch, inn)
            gpu = hip.matvec(wt, x)
            for b in range(batch):
                cpu = port.linear(gtype, w, inn, rows, x[b])
                err = normwise_rel(gpu[b], cpu)
                assert err <= TOL, (rows, inn, batch, b, err)
            say("k-sliced matvec", gtype, rows, inn, batch, "ok")
        wt.release()


def test_k_sliced_matvec_in_a_graph(hip):
    """A batched matvec on the K-sliced kernel captured into a HIP graph
    straight after the upload (its partial-sum scratch was reserved then, so
    the capture allocates nothing): every replay, with eager work and host
    synchronisations between them, equals the eager result bit for bit."""
    import torch
    g = S.rng(4242)
    rows, inn, batch = 2048, 6144, 8
    w = S.quant_matrix(S.Q4_K, rows, inn, g)
    wt = hip.upload(S.Q4_K, inn, rows, w)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(S.normal_f32(g, batch * inn).reshape(batch, inn)).to(dev)
    y = torch.full((batch, rows), float("nan"), device=dev)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        hip.matvec_async(wt, x.data_ptr(), batch, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    eager = torch.empty_like(y)
    with torch.cuda.stream(stream):
        hip.matvec_async(wt, x.data_ptr(), batch, eager.data_ptr(), stream.cuda_stream)
    torch.cuda.synchronize()
    want = eager.cpu().numpy()
    for _ in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    del graph
    wt.release()


@pytest.mark.parametrize("gtype", (S.Q4_K, S.Q6_K, S.Q8_0))
def test_long_matvec_pipelined_rows(hip, port, gtype):
    """Rows enough that every wave walks several row passes (the pipelined
    loop an output head takes: 40,003 rows of 2048, one vector, an odd pass
    count and a partial last pass) against the CPU's linear."""
    g = S.rng(77 + gtype)
    rows, inn = 40003, 2048
    w = S.quant_matrix(gtype, rows, inn, g)
    x = S.normal_f32(g, inn).reshape(1, inn)
    wt = hip.upload(gtype, inn, rows, w)
    gpu = hip.matvec(wt, x)[0]
    cpu = port.linear(gtype, w, inn, rows, x[0])
    err = normwise_rel(gpu, cpu)
    say("long matvec", gtype, "normwise", err)
    assert err <= TOL
    wt.release()


def test_expert_slice_matvec(hip, port):
    layer = S.moe_layer(seed=21, hidden=512, experts=4, ffn=256)
    g = hip.upload(layer.gate_type, 512, 256, layer.gate, n_experts=4)
    d = hip.upload(layer.down_type, 256, 512, layer.down, n_experts=4)
    x = S.normal_f32(S.rng(22), 512)
    a = S.normal_f32(S.rng(23), 256)
    for e in range(4):
        assert normwise_rel(hip.matvec(g, x, expert=e),
                            port.linear(layer.gate_type, layer.gate[e], 512, 256, x)) <= TOL
        assert normwise_rel(hip.matvec(d, a, expert=e),
                            port.linear(layer.down_type, layer.down[e], 256, 512, a)) <= TOL
    with pytest.raises(ValueError):
        hip.matvec(g, x, expert=4)
    g.release()
    d.release()
    # planar types whose slices are padded to 256 bytes between experts
    for gtype in (S.Q4_0, S.Q8_0, S.Q6_K):
        ws = [S.quant_matrix(gtype, 37, 512, S.rng(24 + e)) for e in range(3)]
        wt = hip.upload(gtype, 512, 37, np.concatenate([w.reshape(-1) for w in ws]), n_experts=3)
        for e in range(3):
            assert normwise_rel(hip.matvec(wt, x, expert=e), port.linear(gtype, ws[e], 512, 37, x)) <= TOL
        wt.release()


@pytest.mark.parametrize("gtype", FLOAT + QUANT + QUANT_MORE)
@pytest.mark.parametrize("rows,experts", ((37, 0), (37, 3), (5, 2)))
def test_weight_layout_round_trip(hip, gtype, rows, experts):
    """Q4_0, Q8_0 and Q6_K sit in HBM as per-slice field planes (odd slice
    sizes padded between experts); reading the weight back returns the GGUF
    bytes of every type unchanged."""
    say("round trip", S.TYPE_NAMES[gtype], rows, experts)
    inn = 512
    nbytes = S.row_bytes(gtype, inn) * rows * max(experts, 1)
    w = S.rng(40 + gtype).integers(0, 256, nbytes, dtype=np.uint8)
    wt = hip.upload(gtype, inn, rows, w, experts)
    assert np.array_equal(wt.download(), w)
    wt.release()


def test_try_linear_contract(hip, port):
    from pokitlms_amd.backend import TensorView
    g = S.rng(31)
    w = S.quant_matrix(S.Q4_K, 64, 512, g)
    x = S.normal_f32(g, 512)
    y = np.zeros(64, np.float32)
    assert hip.try_linear(TensorView(S.Q4_K, (512, 64), w), x, y)
    assert normwise_rel(y, port.linear(S.Q4_K, w, 512, 64, x)) <= TOL
    # Q8_K (15) has no kernel: False, so the caller runs its CPU path
    assert not hip.try_linear(TensorView(15, (512, 64), np.zeros(64 * 584, np.uint8)), x, y)
    with pytest.raises(ValueError):
        hip.try_linear(TensorView(S.Q4_K, (512, 64), w), x[:256], y)


# ---- MoE layer ------------------------------------------------------------------------

@pytest.fixture(scope="module")
def c3(hip):
    layer = G.c3_layer()
    handles = hip.upload_moe_layer(layer)
    yield layer, handles
    handles.release()


def test_c3_moe_decode_golden(hip, port, golden, c3):
    layer, h = c3
    toks = G.c3_tokens()
    blk = port.moe(layer)
    hip.reset_stats()
    worst = 0.0
    for t in range(toks.shape[0]):
        y, ids, probs = hip.moe_decode(h, toks[t])
        assert np.array_equal(ids, golden["c3_ids"][t]), (t, ids, golden["c3_ids"][t])
        assert np.max(np.abs(probs - golden["c3_probs"][t])) <= TOL * np.max(golden["c3_probs"][t])
        cpu = golden["c3_y"][t] if t < 4 else blk.forward(toks[t])[0]
        worst = max(worst, normwise_rel(y, cpu))
    say("c3 worst normwise", worst)
    assert worst <= TOL
    # the certified (parallel) routing must carry most tokens; the exact serial
    # path is the exception (it also hid a broken fast path once)
    st = hip.stats()
    say("c3 router fallbacks", st["router_fallbacks"], "of", toks.shape[0])
    assert st["router_fallbacks"] <= toks.shape[0] // 8


def test_c3_moe_reference_order_bit_exact(hip, port, golden, c3):
    """pk_hip_moe_decode_reference_order with the host libm's expf table: the
    reference's ids, probabilities and moe_result bit for bit on all 64
    golden tokens (outputs: the compiled reference's for the first four, the
    oracle -- pinned to it bit for bit -- for the rest)."""
    from pokitlms_amd.model import libm_expf_pairs
    layer, h = c3
    hip.set_libm_expf(libm_expf_pairs())
    try:
        toks = G.c3_tokens()
        blk = port.moe(layer)
        for t in range(toks.shape[0]):
            y, ids, probs = hip.moe_decode_reference_order(h, toks[t])
            assert np.array_equal(ids, golden["c3_ids"][t]), t
            assert np.array_equal(probs.view(np.uint32), golden["c3_probs"][t].view(np.uint32)), t
            cpu = golden["c3_y"][t] if t < 4 else blk.forward(toks[t])[0]
            assert np.array_equal(y.view(np.uint32), cpu.view(np.uint32)), (t, normwise_rel(y, cpu))
    finally:
        hip.set_libm_expf(None)


@pytest.mark.parametrize("gate_type,down_type", ((S.Q5_K, S.Q8_0), (S.Q8_0, S.Q4_K),
                                                 (S.Q4_0, S.Q6_K)))
def test_moe_reference_order_other_formats(hip, port, gate_type, down_type):
    from pokitlms_amd.model import libm_expf_pairs
    layer = S.moe_layer(seed=200 + gate_type, hidden=1024, experts=32, ffn=512, top_k=6,
                        gate_type=gate_type, up_type=gate_type, down_type=down_type)
    h = hip.upload_moe_layer(layer)
    hip.set_libm_expf(libm_expf_pairs())
    try:
        blk = port.moe(layer)
        for i in range(3):
            x = S.normal_f32(S.rng(210 + i), 1024)
            y, ids, probs = hip.moe_decode_reference_order(h, x)
            cy, cids, cprobs = blk.forward(x)
            assert np.array_equal(ids, cids)
            assert np.array_equal(probs.view(np.uint32), cprobs.view(np.uint32))
            assert np.array_equal(y.view(np.uint32), cy.view(np.uint32))
        bad = S.normal_f32(S.rng(219), 1024)
        bad[7] = np.inf
        with pytest.raises(HipError):
            hip.moe_decode_reference_order(h, bad)
        y, _, _ = hip.moe_decode_reference_order(h, x)  # usable after the data error
        assert np.array_equal(y.view(np.uint32), cy.view(np.uint32))
    finally:
        hip.set_libm_expf(None)
        h.release()


def test_moe_decode_deterministic(hip, c3):
    _, h = c3
    x = G.c3_tokens(2)[1]
    y0, i0, p0 = hip.moe_decode(h, x)
    for _ in range(3):
        y1, i1, p1 = hip.moe_decode(h, x)
        assert np.array_equal(bits(y0), bits(y1)) and np.array_equal(i0, i1)
        assert np.array_equal(bits(p0), bits(p1))


def _small_layer(seed, router=None, experts=32, hidden=512, ffn=256, top_k=4, normalize=True):
    layer = S.moe_layer(seed=seed, hidden=hidden, experts=experts, ffn=ffn, top_k=top_k,
                        normalize=normalize)
    if router is not None:
        layer.router = np.ascontiguousarray(router, np.float32)
    return layer


def test_router_ties_break_by_id(hip, port):
    """All-zero router (the reference's smoke models): every logit ties, so
    the routes are experts 0..k-1 with equal weights."""
    layer = _small_layer(50, router=np.zeros((32, 512), np.float32))
    h = hip.upload_moe_layer(layer)
    x = S.normal_f32(S.rng(51), 512)
    y, ids, probs = hip.moe_decode(h, x)
    cy, cids, cprobs = port.moe(layer).forward(x)
    assert np.array_equal(ids, np.arange(4)) and np.array_equal(ids, cids)
    assert np.array_equal(bits(probs), bits(cprobs))
    assert normwise_rel(y, cy) <= TOL
    h.release()


def test_router_near_ties_take_the_exact_path(hip, port):
    """Rows that differ by one ulp in one weight, and exact duplicates: the
    certified ranking cannot separate them, so the exact serial logits decide.
    The ids must still equal the CPU's on every token."""
    g = S.rng(60)
    router = S.normal_f32(g, 32 * 512, 0.02).reshape(32, 512)
    for j in range(0, 32, 2):
        router[j + 1] = router[j]
        k = int(g.integers(0, 512))
        router[j + 1, k] = np.nextafter(router[j, k], np.float32(1))
    layer = _small_layer(61, router=router, top_k=8)
    h = hip.upload_moe_layer(layer)
    blk = port.moe(layer)
    hip.reset_stats()
    for t in range(24):
        x = S.normal_f32(g, 512)
        y, ids, probs = hip.moe_decode(h, x)
        cy, cids, cprobs = blk.forward(x)
        assert np.array_equal(ids, cids), (t, ids, cids)
        assert np.max(np.abs(probs - cprobs)) <= TOL * np.max(cprobs)
        assert normwise_rel(y, cy) <= TOL
    st = hip.stats()
    say("near-tie fallbacks", st["router_fallbacks"], "candidates", st["router_candidates"])
    assert st["router_fallbacks"] > 0
    h.release()


@pytest.mark.parametrize("normalize", (True, False))
def test_moe_shapes_and_normalisation(hip, port, normalize):
    for (hidden, experts, ffn, k, gt, dt) in ((512, 16, 256, 2, S.Q4_K, S.Q6_K),
                                             (1024, 64, 512, 8, S.Q5_K, S.Q8_0),
                                             (2048, 128, 768, 8, S.Q4_0, S.Q4_K),
                                             (1024, 32, 512, 4, S.Q4_1, S.Q4_1)):
        layer = S.moe_layer(seed=70 + hidden, hidden=hidden, experts=experts, ffn=ffn,
                            gate_type=gt, up_type=gt, down_type=dt, top_k=k,
                            normalize=normalize)
        h = hip.upload_moe_layer(layer)
        blk = port.moe(layer)
        for t in range(4):
            x = S.normal_f32(S.rng(700 + t), hidden)
            y, ids, probs = hip.moe_decode(h, x)
            cy, cids, cprobs = blk.forward(x)
            assert np.array_equal(ids, cids)
            assert np.max(np.abs(probs - cprobs)) <= TOL * np.max(cprobs)
            assert normwise_rel(y, cy) <= TOL
        h.release()


@pytest.mark.parametrize("hidden", (512, 1024, 3072))
def test_router_fast_path_widths(hip, port, hidden):
    """Every router width the kernel supports certifies most random tokens
    itself (no exact fallback) and still matches the CPU's routes."""
    layer = S.moe_layer(seed=90 + hidden, hidden=hidden, experts=64, ffn=256, top_k=8)
    h = hip.upload_moe_layer(layer)
    blk = port.moe(layer)
    hip.reset_stats()
    n = 16
    for t in range(n):
        x = S.normal_f32(S.rng(900 + t), hidden)
        y, ids, _ = hip.moe_decode(h, x)
        cy, cids, _ = blk.forward(x)
        assert np.array_equal(ids, cids)
        assert normwise_rel(y, cy) <= TOL
    st = hip.stats()
    say("width", hidden, "fallbacks", st["router_fallbacks"])
    assert st["router_fallbacks"] <= n // 4
    h.release()


def test_non_finite_router_is_a_runtime_error(hip, port):
    from pokitlms_amd.backend import HipError
    router = S.normal_f32(S.rng(80), 32 * 512, 0.02).reshape(32, 512)
    router[5, 7] = np.inf
    layer = _small_layer(81, router=router)
    h = hip.upload_moe_layer(layer)
    with pytest.raises(HipError) as ex:
        hip.moe_decode(h, S.normal_f32(S.rng(82), 512))
    assert ex.value.status == 2 and "non-finite" in str(ex.value)
    h.release()
    # the context stays usable: routing errors are data errors, not device failures
    good = hip.upload_moe_layer(_small_layer(83))
    x = S.normal_f32(S.rng(84), 512)
    y, ids, _ = hip.moe_decode(good, x)
    assert np.array_equal(ids, port.moe(_small_layer(83)).forward(x)[1])
    good.release()


def test_async_device_buffers_match_sync(hip, c3):
    import torch
    _, h = c3
    x = G.c3_tokens(3)[2]
    y_ref, ids_ref, p_ref = hip.moe_decode(h, x)
    dev = torch.device("cuda:0")
    dx = torch.from_numpy(x).to(dev)
    dy = torch.empty(2048, dtype=torch.float32, device=dev)
    di = torch.empty(8, dtype=torch.int32, device=dev)
    dp = torch.empty(8, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    hip.moe_decode_async(h, dx.data_ptr(), dy.data_ptr(), di.data_ptr(), dp.data_ptr(), stream)
    hip.sync(stream)
    assert np.array_equal(bits(dy.cpu().numpy()), bits(y_ref))
    assert np.array_equal(di.cpu().numpy().astype(np.uint32), ids_ref)
    assert np.array_equal(bits(dp.cpu().numpy()), bits(p_ref))


def test_stats_track_resident_experts(hip, c3):
    _, h = c3
    hip.reset_stats()
    hip.moe_decode(h, G.c3_tokens(1)[0])
    st = hip.stats()
    assert st["moe_decode_calls"] == 1 and st["expert_hits"] == 8 and st["expert_misses"] == 0
    assert st["weight_bytes"] == h.routed_bytes() == 25_526_272
    assert st["resident_bytes"] >= h.router.nbytes + h.gate.nbytes + h.up.nbytes + h.down.nbytes


# ---- more layer shapes, near ties at another width, graph replays ------------------------
# (hidden, experts, ffn, top_k, gate/up type, down type)
LAYER_SHAPES = (
    (1024, 64, 512, 8, S.Q4_K, S.Q6_K),
    (2048, 128, 768, 8, S.Q4_K, S.Q4_K),
    (2048, 64, 768, 6, S.Q5_K, S.Q6_K),
    (1024, 32, 256, 4, S.Q8_0, S.Q8_0),
    (4096, 64, 1536, 8, S.Q4_K, S.Q6_K),
)


@pytest.mark.parametrize("shape", LAYER_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}x{s[2]}k{s[3]}t{s[4]}-{s[5]}")
def test_moe_layer_shapes_against_cpu(hip, port, shape):
    hidden, experts, ffn, k, gt, dt = shape
    say("layer shape", shape)
    layer = S.moe_layer(seed=110 + hidden + ffn, hidden=hidden, experts=experts, ffn=ffn,
                        gate_type=gt, up_type=gt, down_type=dt, top_k=k)
    h = hip.upload_moe_layer(layer)
    blk = port.moe(layer)
    for t in range(6):
        x = S.normal_f32(S.rng(1100 + t), hidden)
        y, ids, probs = hip.moe_decode(h, x)
        cy, cids, cprobs = blk.forward(x)
        assert np.array_equal(ids, cids)
        assert np.max(np.abs(probs - cprobs)) <= TOL * np.max(cprobs)
        assert normwise_rel(y, cy) <= TOL
    h.release()


def test_near_ties_at_width_1024(hip, port):
    """Near-tied router rows at a second width: the exact serial ranking
    decides, and the ids equal the CPU's on every token."""
    g = S.rng(130)
    router = S.normal_f32(g, 64 * 1024, 0.02).reshape(64, 1024)
    for j in range(0, 64, 2):
        router[j + 1] = router[j]
        kk = int(g.integers(0, 1024))
        router[j + 1, kk] = np.nextafter(router[j, kk], np.float32(1))
    layer = S.moe_layer(seed=131, hidden=1024, experts=64, ffn=512, top_k=8)
    layer.router = router
    h = hip.upload_moe_layer(layer)
    blk = port.moe(layer)
    hip.reset_stats()
    for t in range(12):
        x = S.normal_f32(g, 1024)
        y, ids, _ = hip.moe_decode(h, x)
        cy, cids, _ = blk.forward(x)
        assert np.array_equal(ids, cids), (t, ids, cids)
        assert normwise_rel(y, cy) <= TOL
    st = hip.stats()
    say("width-1024 near-tie fallbacks", st["router_fallbacks"])
    assert st["router_fallbacks"] > 0
    h.release()


def test_graph_replays_match_eager(hip, c3):
    """A HIP graph of several layers, replayed repeatedly with eager work and
    synchronisation between replays, reproduces the eager results every time
    (no memset node is recorded)."""
    import torch
    _, h = c3
    dev = torch.device("cuda:0")
    xs = torch.from_numpy(G.c3_tokens(4)).to(dev)
    ys = torch.empty(4, 2048, device=dev)
    ids = torch.empty(4, 8, dtype=torch.int32, device=dev)
    ps = torch.empty(4, 8, device=dev)
    stream = torch.cuda.Stream()

    def run(s):
        for t in range(4):
            hip.moe_decode_async(h, xs[t].data_ptr(), ys[t].data_ptr(), ids[t].data_ptr(),
                                 ps[t].data_ptr(), s)
    with torch.cuda.stream(stream):
        run(stream.cuda_stream)
    hip.sync(stream.cuda_stream)
    y_ref, i_ref = ys.clone(), ids.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        ys.zero_()
        ids.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        hip.sync(0)
        assert torch.equal(ys, y_ref) and torch.equal(ids, i_ref), rep
