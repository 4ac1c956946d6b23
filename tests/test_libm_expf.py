"""The libm expf exception table (pokitlms_amd/host/expf_table.c, written at
build time) against this host's libm, called directly through ctypes.

The reference-order decode returns exp-in-double rounded to float except on
the table's inputs, where it returns the table's value; these checks pin that
the pair set is exactly where libm's expf disagrees with that rounding."""
import ctypes

import numpy as np
import pytest

from pokitlms_amd import model as M

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def _expf(bits: np.ndarray) -> np.ndarray:
    xs = bits.view(np.float32)
    return np.array([_libm.expf(float(x)) for x in xs], np.float32)


@pytest.fixture(scope="module")
def pairs():
    try:
        return M.libm_expf_pairs()
    except ImportError as e:
        pytest.skip(str(e))


def test_table_is_sorted_and_one_ulp(pairs):
    assert pairs.shape[0] > 0 and pairs.dtype == np.uint32
    assert np.all(np.diff(pairs[:, 0].astype(np.int64)) > 0)
    x = pairs[:, 0].view(np.float32)
    assert np.all(np.isfinite(x))
    cr = np.exp(x.astype(np.float64)).astype(np.float32)
    ulps = np.abs(cr.view(np.int32).astype(np.int64) - pairs[:, 1].view(np.int32))
    assert np.all(ulps == 1)


def test_table_entries_are_libm_results(pairs):
    rng = np.random.default_rng(0)
    pick = pairs[rng.choice(pairs.shape[0], 4000, replace=False)]
    assert np.array_equal(_expf(pick[:, 0]).view(np.uint32), pick[:, 1])


def test_inputs_outside_table_are_correctly_rounded(pairs):
    rng = np.random.default_rng(1)
    # softmax arguments are <= 0, SwiGLU's -g of either sign: sample both
    x = np.concatenate([rng.uniform(-104.0, 89.0, 60000), rng.uniform(-20.0, 0.0, 60000)])
    bits = x.astype(np.float32).view(np.uint32)
    bits = bits[~np.isin(bits, pairs[:, 0])]
    cr = np.exp(bits.view(np.float32).astype(np.float64)).astype(np.float32)
    assert np.array_equal(_expf(bits).view(np.uint32), cr.view(np.uint32))
