"""The C++ HipLinearBackend (pokitlms_amd/host) inside the reference's own
call sites: tests/native/hip_backend_cases.cpp, built by ``make -C oracle
cases`` against the reference headers and CPU library in place.

On the GPU it runs every case: try_linear through tensor_linear's backend hook
(src/tensor_linear.cpp:213) for every type tensor_linear dispatches (F32/F16/BF16/
Q4_0/Q4_1/Q5_0/Q5_1/Q8_0/Q2_K/Q3_K/Q4_K/Q5_K/Q6_K) against the CPU kernels; false
for a GGUF type without a kernel (Q8_K); shape errors;
file-backed tensors kept resident; the MoE block hook against the reference
MoE block and the Qwen3.5 block with its shared expert (ids exact, outputs
normwise <= 1e-4); a non-finite router as a
data error that leaves the backend usable; two files opened one after the
other with different tensors at one offset (no stale resident copy); the
content-checked LRU set for in-memory tensors; the expert-cache counters; and
the reference's Qwen35Runner driven through set_linear_backend on its dense and
MoE smoke models (tests/golden/qwen35-smoke.gguf and qwen35moe-smoke.gguf,
copies of the reference's tests/data files), whose generate_chat output must
equal the CPU runner's, as in the reference's tests/vulkan_linear_test.cpp:9-36.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CASES = os.path.join(ROOT, "oracle", "_ref", "hip_backend_cases")
RUNNER = os.path.join(ROOT, "oracle", "_ref", "qwen3moe_hip_cases")
RUNNER_MISSING = ("oracle/_ref/qwen3moe_hip_cases is built only where the reference checkout "
                  "is present (make -C oracle runner)")
MISSING = ("oracle/_ref/hip_backend_cases is built only where the reference checkout "
           "is present (make -C oracle cases)")


def _run(*args, timeout):
    r = subprocess.run([CASES, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr[-4000:])
    return r


@pytest.mark.skipif(not os.path.exists(CASES), reason=MISSING)
def test_native_backend_without_a_device_fails_cleanly():
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible; the GPU test covers this host")
    r = _run("--expect-no-device", timeout=60)
    assert r.returncode == 0
    assert r.stdout.startswith("PASS no_device HIP backend:")


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(CASES), reason=MISSING)
def test_native_backend_cases():
    golden = os.path.join(ROOT, "tests", "golden")
    r = _run(os.path.join(golden, "qwen35-smoke.gguf"), os.path.join(golden, "qwen35moe-smoke.gguf"),
             timeout=300)
    assert r.returncode == 0, r.stdout[-3000:]
    lines = r.stdout.splitlines()
    assert not [l for l in lines if l.startswith("FAIL")]
    assert sum(l.startswith("PASS try_linear_parity") for l in lines) == 13
    assert sum(l.startswith("PASS try_linear_unsupported") for l in lines) == 1
    assert sum(l.startswith("PASS moe_block_parity") for l in lines) == 2
    assert sum(l.startswith("PASS moe35_block_parity") for l in lines) == 1
    for name in ("file_reload", "transient_cache", "transient_default", "expert_cache_stats"):
        assert sum(l.startswith("PASS " + name) for l in lines) == 1, name
    assert sum(l.startswith("PASS runner_parity") for l in lines) == 2


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(RUNNER), reason=RUNNER_MISSING)
def test_qwen3moe_runner_selects_hip_backend(tmp_path):
    """The reference's Qwen3MoeRunner with oracle/hip_runner_patch.py's
    set_linear_backend and MoE hook, and the C API's
    pokitlms_qwen3moe_create_with_backend (tests/native/qwen3moe_runner_cases.cpp),
    on the seeded 2-layer model of the whole-model golden: with the
    reference-order HIP backend every greedy token equals the CPU runner's and
    the golden tokens the unpatched reference runner wrote, with the MoE hook
    and try_linear both taking the work; the C API's HIP backend generates the
    CPU backend's text."""
    import numpy as np

    from pokitlms_amd import synth_model as SM
    with np.load(os.path.join(ROOT, "tests", "golden", "model_golden.npz"),
                 allow_pickle=False) as z:
        layers, seed = int(z["small_layers"]), int(z["small_seed"])
        prompt, golden = z["small_prompt"], z["small_tokens"]
    path = str(tmp_path / "small.gguf")
    SM.write_gguf(path, SM.Qwen3MoeShape(layers=layers), seed)
    r = subprocess.run([RUNNER, path, str(len(golden)), *[str(int(t)) for t in prompt]],
                       capture_output=True, text=True, timeout=600)
    print(r.stdout[-6000:])
    print(r.stderr[-3000:])
    assert r.returncode == 0, r.stdout[-3000:]
    lines = r.stdout.splitlines()
    assert not [l for l in lines if l.startswith("FAIL")]
    for name in ("qwen3moe_runner_parity", "backend_reset", "c_api_backend", "c_api_bad_backend"):
        assert sum(l.startswith("PASS " + name) for l in lines) == 1, name
    toks = {l.split()[0]: [int(v) for v in l.split()[1:]] for l in lines
            if l.split() and l.split()[0] in ("cpu_tokens", "hip_tokens")}
    assert toks["cpu_tokens"] == [int(t) for t in golden]
    assert toks["hip_tokens"] == [int(t) for t in golden]
