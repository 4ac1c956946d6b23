"""The router's rounding bound holds for the CPU's serial FP32 sum.

The GPU ranks experts by the FP64 sum S of the CPU's rounded FP32 products
and certifies the order with B = q (2^-24 (1 + 2^-10) + 2^-39), where, for
the chunks of 8 consecutive products (a wave's lanes hold whole chunks),
q = sum_t (8 |O_t| + sum_i |L_{t,i}|) with O_t the sum of the earlier
chunks' products and L_{t,i} the chunk's running sum.  The certified ids are only exact if
|serial FP32 sum - S| <= B always holds; here the serial sum is computed
independently (numpy's sequential float32 cumulative sum, the order of
dot_f32 in src/simd_kernels.hpp:12-24) and the exact value with math.fsum,
on random, heavy-tailed and cancelling rows.
"""
import math

import numpy as np
import pytest


def bound(p: np.ndarray, threads: int = 256) -> float:
    c = p.size // threads
    blocks = p.astype(np.float64).reshape(threads, c)
    offsets = np.concatenate([[0.0], np.cumsum(blocks.sum(axis=1))[:-1]])
    running = np.cumsum(blocks, axis=1)
    q = float(np.sum(c * np.abs(offsets)) + np.sum(np.abs(running)))
    return q * (2.0 ** -24 * (1.0 + 2.0 ** -10) + 2.0 ** -39)


def serial_fp32(p: np.ndarray) -> float:
    return float(np.cumsum(p.astype(np.float32), dtype=np.float32)[-1])


def rows(seed: int, n: int):
    g = np.random.default_rng(seed)
    for k in range(n):
        kind = k % 4
        if kind == 0:  # router-like: N(0, 0.02) weights times N(0, 1) activations
            p = (g.standard_normal(n_el) * 0.02).astype(np.float32) * g.standard_normal(n_el).astype(np.float32)
        elif kind == 1:  # heavy tails
            p = g.standard_cauchy(n_el).astype(np.float32)
        elif kind == 2:  # cancelling: large values followed by their negatives
            big = (g.standard_normal(n_el // 2) * 1e4).astype(np.float32)
            p = np.concatenate([big, -big + g.standard_normal(n_el // 2).astype(np.float32)])
        else:  # a drift that makes the prefix sums large
            p = (g.random(n_el) + 0.5).astype(np.float32)
        yield p.astype(np.float32)


n_el = 2048


@pytest.mark.parametrize("seed", range(3))
def test_serial_sum_within_bound(seed):
    worst = 0.0
    for p in rows(seed, 200):
        exact = math.fsum(float(v) for v in p)
        err = abs(serial_fp32(p) - exact)
        b = bound(p)
        assert err <= b, (err, b)
        worst = max(worst, err / b if b else 0.0)
    assert worst > 0.0  # the rows do exercise rounding


def test_bound_is_not_vacuous():
    """On router-like rows the bound stays small next to the logit spread,
    so most rankings certify without the exact fallback."""
    g = np.random.default_rng(7)
    p = (g.standard_normal(n_el) * 0.02).astype(np.float32) * g.standard_normal(n_el).astype(np.float32)
    spread = 0.02 * math.sqrt(n_el)
    assert bound(p) < 1e-3 * spread


def test_planted_mistake_is_caught():
    """Dropping the offset term (a plausible slip) gives a bound the serial
    sums break on these rows, so the check above can fail."""
    def without_offsets(p, threads=256):
        c = p.size // threads
        q = float(np.sum(np.abs(np.cumsum(p.astype(np.float64).reshape(threads, c), axis=1))))
        return q * (2.0 ** -24 * (1.0 + 2.0 ** -10) + 2.0 ** -39)
    broken = sum(abs(serial_fp32(p) - math.fsum(float(v) for v in p)) > without_offsets(p)
                 for p in rows(0, 200))
    assert broken > 0
