"""Host-side checks of the synthetic skewed-load generator used by the batched
prefill workload (expert load following Zipf(1.1) through a bias-free router)."""
import numpy as np

from pokitlms_amd import synth as S


def test_zipf_targets_cap_and_mass():
    t = S.zipf_targets(512, 128, 8, 1.1)
    assert abs(t.sum() - 4096) < 1e-6
    assert np.all(np.diff(t) <= 1e-9) and t[0] == 512 and np.all(t <= 512)
    # uncapped ranks keep the Zipf ratio
    assert abs(np.log(t[2] / t[3]) / np.log(4 / 3) - 1.1) < 1e-9
    # nothing to cap when the load is flat enough
    flat = S.zipf_targets(512, 128, 1, 0.0)
    assert np.allclose(flat, 4.0)


def test_pinned_direction_keeps_n01():
    u = S.zipf_direction(7, 1024)
    z = S.rng(8).standard_normal((256, 1024))
    x = S.pin_direction(z, u, 1.0)
    assert np.allclose(x.astype(np.float64) @ u, 1.0, atol=1e-4)
    # x - z = (1 - z.u) u: each coordinate moves by at most (1 + |z.u|) |u_i|
    assert np.max(np.abs(x - z)) <= (1 + np.max(np.abs(z @ u))) * np.max(np.abs(u)) + 1e-5
    assert abs(float(x.std()) - 1.0) < 0.02


def test_zipf_router_realises_the_skew():
    """The fitted router, applied to fresh tokens (top-k of exact float64
    logits), gives a load whose exponent is near 1.1 with the top expert
    taken by nearly every token."""
    router, share = S.zipf_router(64, 512, 8, seed=5, calib_tokens=2048, iters=120)
    assert router.shape == (64, 512) and router.dtype == np.float32
    assert abs(share.sum() - 8) < 1e-9
    x = S.zipf_tokens(5, 1024, 512)
    logits = x.astype(np.float64) @ router.astype(np.float64).T
    kth = np.partition(logits, 64 - 8, axis=1)[:, 64 - 8][:, None]
    counts = (logits >= kth).sum(axis=0)
    assert counts.max() >= 0.95 * 1024
    fit = S.zipf_fit(counts)
    assert 0.9 <= fit <= 1.35, fit
    # the realised counts track the targets expert by expert
    expect = share * 1024
    big = expect > 40
    assert np.all(np.abs(counts[big] - expect[big]) <= 0.35 * expect[big] + 10)


def test_zipf_fit_recovers_an_exponent():
    c = np.round(1e5 * np.arange(1, 101, dtype=np.float64) ** -1.3)
    c[0] = c[0] * 2  # a capped head does not enter the fit
    assert abs(S.zipf_fit(c) - 1.3) < 0.01
