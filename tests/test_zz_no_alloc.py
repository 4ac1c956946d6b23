"""pk_hip_moe_decode_noalloc (the decode entry point that allocates nothing:
its scratch is the library's static device array) against
pk_hip_moe_decode_async on the same inputs, through the C ABI: two calls in a
row, the second on a smaller layer, outputs equal bit for bit (the same
kernels in the same order), and the size limit reported as an argument error."""
import numpy as np
import pytest

from pokitlms_amd import synth as S

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _run(hip, handles, x, noalloc):
    import torch
    dev = torch.device("cuda:0")
    k = handles.top_k
    X = torch.from_numpy(x).to(dev)
    Y = torch.full((x.size,), float("nan"), device=dev)
    IDS = torch.full((k,), -1, dtype=torch.int32, device=dev)
    P = torch.full((k,), float("nan"), device=dev)
    fn = hip.moe_decode_noalloc if noalloc else hip.moe_decode_async
    # the fills above run on torch's stream, the call on the library's: let
    # them land first so a late fill cannot overwrite the call's outputs
    torch.cuda.synchronize()
    fn(handles, X.data_ptr(), Y.data_ptr(), IDS.data_ptr(), P.data_ptr())
    hip.sync()
    torch.cuda.synchronize()
    return Y.cpu().numpy(), IDS.cpu().numpy().view(np.uint32), P.cpu().numpy()


def test_noalloc_matches_async_on_two_calls(hip, port):
    # a full config-3 layer, then a smaller one (narrower, fewer experts, top-6)
    shapes = (dict(seed=61, hidden=2048, experts=128, ffn=768, top_k=8),
              dict(seed=62, hidden=1024, experts=64, ffn=512, top_k=6))
    for i, shape in enumerate(shapes):
        say("noalloc call", i, shape)
        layer = S.moe_layer(**shape)
        h = hip.upload_moe_layer(layer)
        x = S.normal_f32(S.rng(shape["seed"] + 100), shape["hidden"])
        y0, ids0, p0 = _run(hip, h, x, noalloc=False)
        y1, ids1, p1 = _run(hip, h, x, noalloc=True)
        assert np.array_equal(ids1, ids0)
        assert np.array_equal(p1.view(np.uint32), p0.view(np.uint32))
        assert np.array_equal(y1.view(np.uint32), y0.view(np.uint32))
        # and the CPU reference: ids exact, outputs within 1e-4 normwise
        cy, cids, _ = port.moe(layer).forward(x)
        assert np.array_equal(ids1, cids)
        assert float(np.max(np.abs(y1 - cy)) / np.max(np.abs(cy))) <= 1e-4
        h.release()


def test_noalloc_rejects_layers_beyond_its_scratch(hip):
    layer = S.moe_layer(seed=63, hidden=512, experts=4, ffn=2560, top_k=2)
    h = hip.upload_moe_layer(layer)
    # INVALID_ARGUMENT (a ValueError in the binding), before any device access
    with pytest.raises(ValueError, match="no-allocation scratch"):
        hip.moe_decode_noalloc(h, 1, 1, 1, 1)
    h.release()
