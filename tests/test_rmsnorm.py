"""RMSNorm exactly as the reference (src/rms_norm.cpp:9-27): the serial FP32
sum of squares, scale = 1 / sqrt(sum / n + eps), out = (x * scale) * w.

The reference-order decode forms the sum of squares without a 2,048-step
dependent chain: inside one binade of the running sum every add rounds to a
fixed grid, so the chain is an integer prefix sum between the steps that tie
(exactly half a grid step) or cross a binade, which are added one by one
(pokitlms_amd/csrc/exact.hip, serial_sum_nonneg).  The CPU tests pin that
algorithm (restated below step for step) against the plain serial sum on rows
built to tie and cross often, and the oracle's rms_norm against the
reference's own (oracle/_ref); the GPU test requires the device result to
equal the oracle's bit for bit through pk_hip_rmsnorm.
"""
import numpy as np
import pytest

F = np.float32


def serial_sum(p):
    s = F(0.0)
    for v in p:
        s = F(s + v)
    return s


def segmented_sum(p):
    """serial_sum_nonneg of exact.hip, step for step in float32 (chunks of 256,
    four values per lane, the wave's scan as a cumulative sum, the first lane
    that ties, meets a non-finite value or crosses the binade added serially)."""
    p = np.asarray(p, F)
    n = p.size
    t = min(n, 64)
    s = serial_sum(p[:t])
    top = 1 << 24
    while t < n:
        e = int((np.frombuffer(s.tobytes(), np.uint32)[0] >> 23) & 0xff) - 127
        if not (s > 0) or not np.isfinite(s) or e < -100 or e > 100:
            s = F(s + p[t])
            t += 1
            continue
        inv_u = F(2.0) ** (23 - e)
        u = F(2.0) ** (e - 23)
        a = int(F(s * inv_u))
        incl = 0
        stop_lane = None
        for L in range(64):
            c = 0
            stop = False
            for i in range(4):
                idx = t + 4 * L + i
                x = p[idx] if idx < n else F(0.0)
                q = F(x * inv_u)
                r = np.rint(q)
                stop = stop or abs(F(q - r)) == F(0.5) or not (x < np.inf)
                c += int(np.fmin(r, F(16777216.0)))
            c = min(c, top)
            if stop or a + incl + c >= top:
                stop_lane = (L, incl)
                break
            incl += c
        if stop_lane is None:
            s = F(F(a + incl) * u)
            t = min(t + 256, n)
        else:
            L, before = stop_lane
            s = F(F(a + before) * u)
            b = t + 4 * L
            for idx in range(b, min(b + 4, n)):
                s = F(s + p[idx])
            t = min(b + 4, n)
    return s


def adversarial_rows(seed=0):
    """(name, row) pairs: random, tie-heavy dyadic values, wide ranges, zeros,
    exact binade boundaries, tiny (subnormal squares) and huge values."""
    g = np.random.default_rng(seed)
    rows = []
    for n in (1, 2, 63, 64, 65, 255, 256, 257, 300, 1000, 2048, 4096):
        rows.append((f"normal{n}", g.standard_normal(n).astype(F)))
    for n in (300, 2048):
        rows.append((f"dyadic{n}", (g.integers(-64, 64, n) / 8.0).astype(F)))
        rows.append((f"dyadic_fine{n}", (g.integers(-4096, 4096, n) / 512.0).astype(F)))
        rows.append((f"wide{n}", (g.standard_normal(n) * 2.0 ** g.integers(-30, 30, n)).astype(F)))
        rows.append((f"ones{n}", np.ones(n, F)))
        z = np.zeros(n, F)
        z[g.integers(0, n, 5)] = g.standard_normal(5)
        rows.append((f"sparse{n}", z))
        big = (g.standard_normal(n) * 1e-3).astype(F)
        big[0] = F(1000.0)
        rows.append((f"big_first{n}", big))
        rows.append((f"tiny{n}", (g.standard_normal(n) * 1e-24).astype(F)))
        rows.append((f"huge{n}", (g.standard_normal(n) * 1e18).astype(F)))
        half = np.full(n, F(2.0 ** -12))  # each square is half an ulp of 1.0: every step ties
        half[0] = F(1.0)
        rows.append((f"halfulp{n}", half))
    rows.append(("zeros", np.zeros(700, F)))
    return rows


@pytest.mark.parametrize("name,row", adversarial_rows(), ids=lambda v: v if isinstance(v, str) else "")
def test_segmented_sum_equals_serial_chain(name, row):
    sq = (row * row).astype(F)
    assert np.array_equal(np.array([segmented_sum(sq)], F).view(np.uint32),
                          np.array([serial_sum(sq)], F).view(np.uint32)), name


def test_segmented_sum_random_lengths():
    g = np.random.default_rng(5)
    for trial in range(40):
        n = int(g.integers(1, 1500))
        row = (g.standard_normal(n) * 2.0 ** g.integers(-8, 8)).astype(F)
        if trial % 3 == 0:
            row = (np.round(row * 16) / 16).astype(F)
        sq = (row * row).astype(F)
        assert segmented_sum(sq) == serial_sum(sq), (trial, n)


def test_oracle_rms_norm_is_the_definition(port):
    g = np.random.default_rng(1)
    x = g.standard_normal((3, 513)).astype(F)
    w = g.standard_normal(513).astype(F)
    out = port.rms_norm(x, w, 1e-6)
    for r in range(3):
        s = serial_sum((x[r] * x[r]).astype(F))
        scale = F(F(1.0) / np.sqrt(F(s / F(513)) + F(1e-6)))
        want = ((x[r] * scale).astype(F) * w).astype(F)
        assert np.array_equal(out[r].view(np.uint32), want.view(np.uint32))


def test_oracle_rms_norm_matches_reference():
    import oracle
    if not oracle.available("reference"):
        pytest.skip("oracle/_ref not built")
    port, ref = oracle.Oracle("port"), oracle.Oracle("reference")
    for name, row in adversarial_rows(2):
        if not np.all(np.isfinite(row * row)):
            continue
        w = np.linspace(-2, 2, row.size).astype(F)
        a, b = port.rms_norm(row, w, 1e-5), ref.rms_norm(row, w, 1e-5)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name


@pytest.mark.gpu
def test_gpu_rmsnorm_bit_exact(hip, port):
    for name, row in adversarial_rows(3):
        w = np.random.default_rng(row.size).standard_normal(row.size).astype(F)
        for eps in (1e-6, 1e-5):
            got = hip.rmsnorm(row, w, eps)
            want = port.rms_norm(row, w, eps)
            if np.all(np.isfinite(want)):
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
            else:
                assert np.array_equal(np.isnan(got), np.isnan(want)), name
    # many rows in one call
    x = np.random.default_rng(9).standard_normal((37, 2048)).astype(F)
    w = np.random.default_rng(10).standard_normal(2048).astype(F)
    assert np.array_equal(hip.rmsnorm(x, w, 1e-6).view(np.uint32),
                          port.rms_norm(x, w, 1e-6).view(np.uint32))


@pytest.mark.gpu
def test_gpu_rmsnorm_rejects_bad_widths(hip):
    with pytest.raises(ValueError):
        hip.rmsnorm(np.ones(8193, F), np.ones(8193, F), 1e-6)
