"""The traced MoE decode (pk_hip_moe_decode_traced_async): the same outputs,
bit for bit, as the untraced call, and per wave phase stamps that are
present for every wave that ran and never decrease along a kernel's phases."""
import numpy as np
import pytest

from pokitlms_amd import _abi
from pokitlms_amd import synth as S

pytestmark = pytest.mark.gpu


def test_traced_decode_equals_untraced_and_stamps_are_ordered(hip):
    import torch
    dev = torch.device("cuda:0")
    layer = S.moe_layer(seed=91)
    h = hip.upload_moe_layer(layer)
    try:
        x = torch.from_numpy(S.normal_f32(S.rng(92), 2048)).to(dev)
        outs = []
        trace = torch.zeros(_abi.TRACE_WORDS, dtype=torch.int64, device=dev)
        for traced in (False, True):
            y = torch.zeros(2048, device=dev)
            ids = torch.zeros(8, dtype=torch.int32, device=dev)
            p = torch.zeros(8, device=dev)
            torch.cuda.synchronize()
            if traced:
                hip.moe_decode_traced_async(h, x.data_ptr(), y.data_ptr(), ids.data_ptr(),
                                            p.data_ptr(), trace.data_ptr())
            else:
                hip.moe_decode_async(h, x.data_ptr(), y.data_ptr(), ids.data_ptr(), p.data_ptr())
            hip.sync()
            torch.cuda.synchronize()
            outs.append((y.cpu().numpy(), ids.cpu().numpy(), p.cpu().numpy()))
        for a, b in zip(*outs):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        t = trace.cpu().numpy().reshape(3, 8192, 8)
        slots = (3, 5, 5)
        waves = (128, 768 * 4, 512 * 8)  # router rows, gate/up and down workgroups' waves
        for k in range(3):
            live = t[k, :, 0] > 0
            assert int(live.sum()) == waves[k], (k, int(live.sum()))
            st = t[k, live, :slots[k]]
            assert (np.diff(st, axis=1) >= 0).all(), k
            assert not t[k, ~live].any()
        # the kernels run in order
        assert t[1, :, 0][t[1, :, 0] > 0].min() >= t[0, :, 0][t[0, :, 0] > 0].min()
        assert t[2, :, 0][t[2, :, 0] > 0].min() >= t[1, :, 0][t[1, :, 0] > 0].min()
    finally:
        h.release()
