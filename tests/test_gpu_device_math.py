"""The two device facts the reference-order decode relies on, checked
exhaustively on the GPU through the C ABI:

* the device's binary16 -> binary32 decode (every fp16 scale and F16 weight
  goes through it) equals the reference's half_to_float
  (src/quantized_linear.cpp:18-39, restated as pko_half_to_float and pinned
  against numpy on the CPU) on all 65,536 bit patterns, NaN payloads aside
  (both give a NaN);
* the device's expf of the reference-order decode (the exponential in double
  rounded once, replaced from the exception table libm_expf.bin) equals this
  host's libm expf, which the reference's softmax and SwiGLU call
  (src/kv_cache.cpp:249, src/qwen3_moe_runner.cpp:683), on every float in
  [-104, 89] (in blocks of bit patterns covering [-112, 96)), compared as block
  checksums that the host recomputes with its own expf.

Also: the device's row decode of every quantized type equals the rows the
compiled reference's dequantize_quantized_row wrote into the golden file.
"""
import numpy as np
import pytest

from pokitlms_amd import synth as S
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu

QUANT_ALL = (S.Q4_0, S.Q4_1, S.Q5_0, S.Q5_1, S.Q8_0, S.Q2_K, S.Q3_K, S.Q4_K, S.Q5_K, S.Q6_K)


def say(*a):
    print(*a, flush=True)


def test_half_decode_exhaustive(hip, port):
    patterns = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    w = hip.upload(S.F16, 65536, 1, patterns.view(np.uint8))
    got = hip.dequantize_rows(w)[0]
    w.release()
    want = np.array([port.half_to_float(int(b)) for b in patterns], dtype=np.float32)
    nan = np.isnan(want)
    assert int(nan.sum()) == 2 * 1023  # the binary16 NaN encodings
    assert np.array_equal(np.isnan(got), nan)
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    assert np.array_equal(gb[~nan], wb[~nan])  # signed zeros, subnormals, infinities included
    say("fp16 decode: 65,536 patterns equal,", int(nan.sum()), "NaNs")


@pytest.mark.parametrize("gtype", QUANT_ALL)
def test_row_decode_equals_reference_rows(hip, port, golden, gtype):
    w, _, inn = G.small_inputs(gtype)
    wt = hip.upload(gtype, inn, 37, w)
    rows = hip.dequantize_rows(wt)
    wt.release()
    # the compiled reference's own dequantize_quantized_row of row 0
    key = f"small_{S.TYPE_NAMES[gtype]}_row0"
    assert np.array_equal(rows[0].view(np.uint32), golden[key].view(np.uint32))
    for r in (17, 36):
        want = port.dequantize_row(gtype, w[r], inn)
        assert np.array_equal(rows[r].view(np.uint32), want.view(np.uint32)), r


def test_row_decode_of_expert_slices(hip, port):
    g = S.rng(91)
    for gtype in (S.Q6_K, S.Q3_K, S.Q4_K):
        ws = [S.quant_matrix(gtype, 13, 512, g) for _ in range(3)]
        wt = hip.upload(gtype, 512, 13, np.concatenate([w.reshape(-1) for w in ws]), n_experts=3)
        for e in range(3):
            got = hip.dequantize_rows(wt, 5, 4, expert=e)
            for r in range(4):
                want = port.dequantize_row(gtype, ws[e][5 + r], 512)
                assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), (gtype, e, r)
        wt.release()


def test_expf_matches_host_libm_on_every_float_in_range(hip, port):
    from pokitlms_amd.model import libm_expf_pairs
    pairs = libm_expf_pairs()
    say("libm exception pairs:", pairs.shape[0])
    block = 1 << 20
    # [+0, 96.0) and [-0, -112.0): 0x42C00000 and 0x42E00000 are multiples of 2^20
    for first, n_blocks in ((0x00000000, 0x42C00000 // block), (0x80000000, 0x42E00000 // block)):
        dev = hip.expf_block_sums(pairs, first, block, n_blocks)
        host = port.expf_block_sums(first, block, n_blocks)
        bad = np.nonzero(dev != host)[0]
        say(f"expf blocks from {first:#010x}: {n_blocks} blocks of 2^20, {bad.size} differ")
        assert bad.size == 0, [hex(first + int(k) * block) for k in bad[:8]]
    # without the table the device returns the correctly rounded exponential,
    # which differs from libm somewhere in a block that holds an exception
    k = (int(pairs[0, 0]) - 0x80000000) // block if pairs[0, 0] >= 0x80000000 else int(pairs[0, 0]) // block
    first = (0x80000000 if pairs[0, 0] >= 0x80000000 else 0) + k * block
    assert hip.expf_block_sums(np.zeros((0, 2), np.uint32), first, block, 1)[0] != \
        port.expf_block_sums(first, block, 1)[0]
