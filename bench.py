#!/usr/bin/env python3
"""Headline benchmark: single-token Qwen3-MoE layer decode on one MI355X.

Workload: hidden 2048, 128 experts, top-8 softmax
routing renormalised; F32 router 2048x128 N(0, 0.02); experts gate/up
2048->768 Q4_K and down 768->2048 Q6_K; SwiGLU; weighted combine; x ~ N(0, 1).

A step is one MoE-layer pass for one token: router + top-k, gate/up SwiGLU,
down + combine (three kernels).  Weights are resident in HBM; every step
reads a different one of --layers distinct layers (24 x 392 MB) with a
different token, so the routed 25.5 MB never comes from the 256 MB MALL.
The timed steps run as HIP-graph replays on one stream (the launch cost of
three ~microsecond kernels would otherwise dominate); eager timing is
reported beside it.

value = algorithmic bytes of the timed steps / wall time, where one step's
algorithmic bytes are the router (1,048,576 B) plus the 8 selected experts'
gate, up and down slices (8 x 3,059,712 B): 25,526,272 B.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "MoE-layer decode achieved HBM GB/s (% of peak); model decode tokens/sec"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--graph-chunk", type=int, default=250)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of graphs")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched-prefill leg")
    ap.add_argument("--prefill-reps", type=int, default=40)
    ap.add_argument("--no-decode", action="store_true", help="skip the whole-model decode leg")
    ap.add_argument("--no-matvec", action="store_true", help="skip the C1/C2 matvec leg")
    ap.add_argument("--no-floor", action="store_true", help="skip the plain-read floor leg")
    ap.add_argument("--timeline", action="store_true",
                    help="only the per-phase timeline of a step (prints JSON and a table)")
    ap.add_argument("--matvec-reps", type=int, default=10)
    ap.add_argument("--decode-cpu-full", action="store_true",
                    help="only time the reference CPU runner on the full 48-layer model")
    ap.add_argument("--matvec-only", action="store_true",
                    help="run only the C1/C2 matvec leg (prints its JSON)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB three times "
                         "(the known-size kernel that scales rocprofv3 FETCH/WRITE_SIZE)")
    return ap.parse_args()


def cpu_info() -> dict:
    """The host CPU model (/proc/cpuinfo) and the threads this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "nproc": usable}


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled), or None."""
    path = os.path.join(ROOT, "profiles", "moe_layer_decode_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == kernel and parts[1] == "traffic_bytes":
                    return int(parts[2])
    except OSError:
        pass
    return None


def device_quant(torch, gtype, rows, inn, gen, dev):
    """GGUF-encoded random weights made on the GPU: uniform quant bytes,
    fp16 scales |N(0, 0.02)| (the same recipe as pokitlms_amd.synth)."""
    from pokitlms_amd import synth as S
    bb = S.BLOCK_BYTES[gtype]
    nb = rows * inn // S.BLOCK_ELEMENTS[gtype]
    blocks = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=dev, generator=gen)
    for off in S.SCALE_OFFSETS[gtype]:
        h = (torch.randn(nb, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
        blocks[:, off:off + 2] = h.view(torch.uint8).view(nb, 2)
    return blocks.view(-1)


def build_layers(torch, hip, n_layers, dev, hidden=2048, experts=128, ffn=768):
    from pokitlms_amd import synth as S
    from pokitlms_amd.backend import MoeLayerHandles
    layers = []
    for li in range(n_layers):
        gen = torch.Generator(device=dev)
        gen.manual_seed(1000 + li)
        router = (torch.randn(experts * hidden, device=dev, generator=gen) * 0.02).contiguous()
        r = hip.upload_device(S.F32, hidden, experts, router.data_ptr(), router.numel() * 4)
        del router
        parts = []
        for gtype, inn, out in ((S.Q4_K, hidden, ffn), (S.Q4_K, hidden, ffn), (S.Q6_K, ffn, hidden)):
            buf = device_quant(torch, gtype, experts * out, inn, gen, dev)
            parts.append(hip.upload_device(gtype, inn, out, buf.data_ptr(), buf.numel(), experts))
            del buf
        layers.append(MoeLayerHandles(r, *parts, top_k=8, normalize=True))
        torch.cuda.synchronize()
    return layers


PREFILL_TOKENS = 512
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA; the prefill GEMMs run on it
MFMA_F32_PEAK_TFLOPS = 157.3
SPLIT_PASSES = 3  # activations as three exact bf16 parts: three MFMA passes per product
# 512 tokens x 8 routes x (gate + up + down: 3 x 2 x 2048 x 768 flops) + router 512 x 128 x 2 x 2048
PREFILL_FLOPS = PREFILL_TOKENS * 8 * 9_437_184 + PREFILL_TOKENS * 128 * 2 * 2048
PREFILL_GEMM_FLOPS = {"gate_up": PREFILL_TOKENS * 8 * 2 * 2 * 2048 * 768,
                      "down": PREFILL_TOKENS * 8 * 2 * 768 * 2048}


def prefill_leg(torch, hip, layers, stream, reps: int, with_cpu: bool):
    """Batched prefill: 512 tokens through the config-3
    layer shape with a router fitted so the expert load follows Zipf(1.1).
    The rotated layers keep their expert weights; each gets the fitted router.
    Timed as `reps` back-to-back prefills on one stream (HIP events), then
    once more per phase with the library's own launch-stream events."""
    import numpy as np

    from pokitlms_amd import synth as S
    from pokitlms_amd.backend import MoeLayerHandles

    router, _ = S.zipf_router(128, 2048, 8, seed=404)
    x = S.zipf_tokens(404, PREFILL_TOKENS, 2048)
    dev = torch.device("cuda:0")
    r = hip.upload(S.F32, 2048, 128, router)
    zl = [MoeLayerHandles(r, l.gate, l.up, l.down, top_k=8, normalize=True) for l in layers]
    X = torch.from_numpy(x).to(dev)
    Y = torch.empty(PREFILL_TOKENS, 2048, device=dev)
    IDS = torch.empty(PREFILL_TOKENS, 8, dtype=torch.int32, device=dev)
    P = torch.empty(PREFILL_TOKENS, 8, device=dev)

    def run(i, s):
        hip.moe_prefill_async(zl[i % len(zl)], X.data_ptr(), PREFILL_TOKENS, Y.data_ptr(),
                              IDS.data_ptr(), P.data_ptr(), s)
    with torch.cuda.stream(stream):
        s = stream.cuda_stream
        for i in range(3):
            run(i, s)
        hip.sync(s)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for i in range(reps):
            run(i, s)
        ev1.record(stream)
        ev1.synchronize()
        hip.sync(s)
        ms = ev0.elapsed_time(ev1) / reps
    # per-phase device time (k_hold keeps host launch gaps out of the events)
    hip.reset_stats()
    hip.set_kernel_timing(True)
    n = 10
    with torch.cuda.stream(stream):
        for i in range(n):
            run(i, stream.cuda_stream)
    hip.set_kernel_timing(False)
    st = hip.stats()
    phase_us = {k: st[f"prefill_{k}_ns"] / n / 1e3 for k in ("route", "gate_up", "down")}
    # parity: every token's routes equal the single-token decode path's, outputs
    # within 1e-4 normwise (the decode path is itself checked against the CPU)
    hip.moe_prefill_async(zl[0], X.data_ptr(), PREFILL_TOKENS, Y.data_ptr(), IDS.data_ptr(),
                          P.data_ptr(), stream.cuda_stream)
    hip.sync(stream.cuda_stream)
    y, ids = Y.cpu().numpy(), IDS.cpu().numpy().astype(np.uint32)
    worst, ids_ok = 0.0, True
    for t in range(0, PREFILL_TOKENS, 4):
        dy, dids, _ = hip.moe_decode(zl[0], x[t])
        ids_ok = ids_ok and bool(np.array_equal(dids, ids[t]))
        worst = max(worst, float(np.max(np.abs(dy - y[t])) / np.max(np.abs(dy))))
    counts = np.bincount(ids.ravel().astype(np.int64), minlength=128)
    gu_tflops = PREFILL_GEMM_FLOPS["gate_up"] / (phase_us["gate_up"] * 1e-6) / 1e12
    # rows the 32-row tiles issue per assignment (partly filled last tiles)
    tile_padding = float(np.sum(32 * ((counts + 31) // 32))) / float(counts.sum())
    whole_tflops = PREFILL_FLOPS / (ms * 1e-3) / 1e12
    out = {
        "workload": "512 tokens x ~ N(0,1) (one direction pinned) through the config-3 layer; "
                    "router fitted so the expert load follows Zipf(1.1)",
        "ms_per_batch": round(ms, 4),
        "tokens_per_s": round(PREFILL_TOKENS / (ms * 1e-3), 1),
        "flops_per_batch": PREFILL_FLOPS,
        "tflops": round(whole_tflops, 2),
        "roofline": {"bound": "mfma",
                     "kernel": "k_expert_gemm<Q4_K, gate/up> (v_mfma_f32_32x32x16_bf16)",
                     "achieved": round(gu_tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gu_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     # issued = algorithmic x three bf16 planes x tile padding
                     "mfma_issued_tflops": round(SPLIT_PASSES * tile_padding * gu_tflops, 2),
                     "tile_padding": round(tile_padding, 3),
                     "frac_of_fp32_mfma_peak": round(gu_tflops / MFMA_F32_PEAK_TFLOPS, 4),
                     "avg_us": round(phase_us["gate_up"], 2),
                     "algorithmic_flops": PREFILL_GEMM_FLOPS["gate_up"]},
        "phase_us": {k: round(v, 2) for k, v in phase_us.items()},
        # the roofline as flat fields too (nested objects are not kept by every reader)
        "gate_up_tflops": round(gu_tflops, 2),
        "gate_up_frac_of_bf16_peak": round(gu_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "gate_up_us": round(phase_us["gate_up"], 2),
        "down_us": round(phase_us["down"], 2),
        "route_us": round(phase_us["route"], 2),
        "ids_equal_decode": ids_ok,
        "normwise_vs_decode": worst,
        "router_fallbacks_per_batch": st["router_fallbacks"] / n,
        "router_candidates_per_batch": st["router_candidates"] / n,
        "expert_load": {"max": int(counts.max()), "touched": int((counts > 0).sum()),
                        "zipf_fit": round(S.zipf_fit(counts), 3)},
        "parity_vs_decode": {"ids_equal": ids_ok, "normwise_rel": worst, "tokens": 128},
        "layers_rotated": len(zl),
    }
    if with_cpu:
        log("prefill cpu baseline (512 single-token reference MoE blocks) ...")
        cpu = prefill_cpu_baseline()
        out["cpu_baseline"] = cpu
        out["cpu_tokens_per_s"] = cpu["tokens_per_s"]
        out["speedup_vs_cpu"] = round(out["tokens_per_s"] / cpu["tokens_per_s"], 1)
    r.release()
    return out


# Plain-read floors: the whole config-3 step's routed bytes, each of its two
# expert kernels' bytes, and config 1's matrix.
FLOOR_BYTES = {"step": 25_526_272, "gate_up": 14_188_544, "down": 10_354_688,
               "c1": 9_437_184}


def floor_leg(torch, hip, stream, reps: int = 20):
    """What a plain streaming read (pk_hip_read_floor_async: 16-byte
    nontemporal loads over the whole chip) takes for each byte count, timed
    like the MoE step: a HIP graph of one launch per distinct copy (at least
    640 MB of copies, so nothing is served from the 256 MB MALL), replayed
    `reps` times; per-launch time = graph time / launches."""
    dev = torch.device("cuda:0")
    out = {}
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    for name, nbytes in FLOOR_BYTES.items():
        copies = max(4, -(-(640 << 20) // nbytes))
        buf = torch.randint(0, 256, (copies * nbytes,), dtype=torch.uint8, device=dev)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            cs = torch.cuda.current_stream().cuda_stream
            for c in range(copies):
                hip.read_floor_async(buf.data_ptr() + c * nbytes, nbytes, sink.data_ptr(), cs)
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            for _ in range(reps):
                g.replay()
            ev1.record(stream)
            ev1.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / (reps * copies)
        out[name] = {"bytes": nbytes, "us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "copies": copies}
        log(f"read floor {name} {nbytes} B: {us:.3f} us/launch, {nbytes / us / 1e3:.0f} GB/s")
        del g, buf
        torch.cuda.synchronize()
    return out


def prefill_cpu_baseline(kind_pref: str = "reference"):
    """The reference MoE block (oracle/_ref, its row pool; the port when the
    reference library is absent) run on the 512 config-4 tokens one at a time,
    as the reference prefills (src/qwen3_moe_runner.cpp:785-790), through a
    config-3 layer with the fitted Zipf router: total wall seconds."""
    import oracle
    from pokitlms_amd import synth as S
    kind = kind_pref if oracle.available(kind_pref) else "port"
    cpu = oracle.Oracle(kind)
    layer = S.moe_layer(seed=3)
    router, _ = S.zipf_router(128, 2048, 8, seed=404)
    layer.router = router
    blk = cpu.moe(layer)
    x = S.zipf_tokens(404, PREFILL_TOKENS, 2048)
    blk.forward(x[0])  # warm-up
    t0 = time.perf_counter()
    for t in range(PREFILL_TOKENS):
        blk.forward(x[t])
    secs = time.perf_counter() - t0
    cores = cpu.lib.pkref_row_workers() if kind == "reference" else 1
    return {"tokens_per_s": round(PREFILL_TOKENS / secs, 2), "seconds": round(secs, 3),
            "cores": int(cores), "kind": kind, **cpu_info(),
            "sample": f"{PREFILL_TOKENS} config-4 tokens through the reference MoE block one "
                      f"at a time (Zipf router fitted as the GPU leg's), row pool of {cores}"}


MATVEC_COPIES = 64  # distinct weight copies per case (at most; > 2x the 256 MB MALL)


def matvec_cases():
    """BASELINE configs[0] (Q4_K 4096x4096, one vector) and configs[1] (five
    formats at 2048x6144 and 6144x2048, out x in, batches of 1, 4 and 8)."""
    from pokitlms_amd import synth as S
    cases = [("c1", S.Q4_K, 4096, 4096, 1)]
    for t in (S.Q4_0, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K):
        for out, inn in ((2048, 6144), (6144, 2048)):
            for b in (1, 4, 8):
                cases.append(("c2", t, out, inn, b))
    # the config-5 model's Q6_K output head (151936 x 2048, 255 MB), one vector
    cases.append(("c5_head", S.Q6_K, 151936, 2048, 1))
    return cases


def matvec_cpu_us(cpu, gtype, rows, inn, batch, seed, reps: int = 5):
    """The reference tensor_linear (oracle/_ref, row pool of min(6, max(2,
    nproc - 1)) workers, src/tensor_linear.cpp:20-128,196-227) on one random
    matrix of the case's format and shape: `batch` calls per timed rep (the
    reference has no batched matvec), median of `reps` reps after one warm-up
    call, in microseconds per rep."""
    import numpy as np

    from pokitlms_amd import synth as S
    g = S.rng(seed)
    w = S.quant_matrix(gtype, rows, inn, g)
    x = S.normal_f32(g, inn)
    cpu.linear_repeat(gtype, w, inn, rows, x, 1)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cpu.linear_repeat(gtype, w, inn, rows, x, batch)
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e6


def matvec_leg(torch, hip, stream, reps: int, only=None, with_cpu: bool = True):
    """K-quant matvec throughput (configs[0..1]).  Each case's weights are one
    expert tensor of MATVEC_COPIES distinct random matrices made on the GPU;
    a HIP graph launches the matvec once per copy, so the weights stream from
    HBM, and replays `reps` times (per-launch time = graph time / launches,
    inter-kernel gaps included).  The library's launch-stream events then
    time 64 single launches (each queued behind a hold kernel), which is the
    kernel's own duration plus its dispatch.  GB/s counts the algorithmic
    bytes: the weights once plus 4 * batch * (in + out)."""
    from pokitlms_amd import synth as S
    dev = torch.device("cuda:0")
    out = []
    cpu = None
    if with_cpu:
        import oracle
        if oracle.available("reference"):
            cpu = oracle.Oracle("reference")
    for name, gtype, rows, inn, batch in matvec_cases():
        if only and (S.TYPE_NAMES[gtype], rows, inn, batch) not in only:
            continue
        gen = torch.Generator(device=dev)
        gen.manual_seed(5000 + gtype * 64 + batch + (rows // 2048))
        copies = max(4, min(MATVEC_COPIES, (1 << 31) // S.matrix_bytes(gtype, inn, rows)))
        buf = device_quant(torch, gtype, copies * rows, inn, gen, dev)
        w = hip.upload_device(gtype, inn, rows, buf.data_ptr(), buf.numel(), copies)
        del buf
        X = torch.randn(batch, inn, device=dev, generator=gen)
        Y = torch.empty(copies, batch, rows, device=dev)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            cs = torch.cuda.current_stream().cuda_stream
            for e in range(copies):
                hip.matvec_async(w, X.data_ptr(), batch, Y[e].data_ptr(), cs, expert=e)
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            for _ in range(reps):
                g.replay()
            ev1.record(stream)
            ev1.synchronize()
        us_graph = ev0.elapsed_time(ev1) * 1e3 / (reps * copies)
        hip.reset_stats()
        hip.set_kernel_timing(True)
        with torch.cuda.stream(stream):
            for e in range(copies):
                hip.matvec_async(w, X.data_ptr(), batch, Y[e].data_ptr(),
                                 stream.cuda_stream, expert=e)
        hip.set_kernel_timing(False)
        st = hip.stats()
        us_event = st["matvec_ns"] / st["matvec_launches"] / 1e3
        nbytes = S.matrix_bytes(gtype, inn, rows) + 4 * batch * (inn + rows)
        rec = {"config": name, "type": S.TYPE_NAMES[gtype], "out": rows, "in": inn,
               "batch": batch, "bytes": nbytes, "copies": copies,
               "us_graph": round(us_graph, 3), "us_event": round(us_event, 3),
               "gbs_graph": round(nbytes / us_graph / 1e3, 1),
               "gbs_event": round(nbytes / us_event / 1e3, 1),
               "frac_event": round(nbytes / us_event / 1e3 / HBM_PEAK_GBS, 4)}
        if cpu is not None:
            cpu_us = matvec_cpu_us(cpu, gtype, rows, inn, batch, 7000 + gtype + rows // 2048)
            rec["cpu_us"] = round(cpu_us, 1)
            rec["speedup_vs_cpu"] = round(cpu_us / us_graph, 1)
        out.append(rec)
        log(f"matvec {name} {S.TYPE_NAMES[gtype]} {rows}x{inn} B={batch}: "
            f"{us_graph:.2f} us/launch (graph), {us_event:.2f} us (event), "
            f"{nbytes / us_graph / 1e3:.0f} GB/s"
            + (f", cpu {rec['cpu_us']:.0f} us" if cpu is not None else ""))
        del g, X, Y
        w.release()
        torch.cuda.synchronize()
    return out


def decode_weight_bytes(shape) -> int:
    """Algorithmic weight bytes of one decode forward: every dense tensor,
    top_k of the n_experts slices of each expert tensor, one embedding row."""
    from pokitlms_amd import gguf
    from pokitlms_amd import synth_model as SM
    total = 0
    for name, dims, gtype, _ in SM.tensor_list(shape):
        nbytes = gguf.payload_bytes(gtype, dims)
        if name == "token_embd.weight":
            total += nbytes // dims[1]
        elif "_exps." in name:
            total += nbytes // shape.experts * shape.top_k
        else:
            total += nbytes
    return total


def decode_cpu_baseline(prompt_len: int = 32, forwards: int = 20):
    """The reference Qwen3MoeRunner (oracle/_ref) on models of the config-5
    shape with 1 and 4 layers (GGUF files in /dev/shm, all experts cached after
    the prompt), steady-state seconds per forward extrapolated linearly to 48
    layers: t(L) = head + L * layer."""
    import numpy as np

    import oracle
    from pokitlms_amd import synth_model as SM
    if not oracle.available("reference"):
        return None
    cpu = oracle.Oracle("reference")
    d = "/dev/shm" if os.path.isdir("/dev/shm") else "/tmp"
    med = {}
    for L in (1, 4):
        m = SM.Qwen3MoeShape(layers=L)
        path = os.path.join(d, f"pk_bench_decode_{os.getpid()}_{L}.gguf")
        try:
            SM.write_gguf(path, m, 1234)
            secs = cpu.qwen3moe_forward_times(path, SM.prompt_tokens(1234, prompt_len, m.vocab),
                                              forwards)
        finally:
            if os.path.exists(path):
                os.remove(path)
        med[L] = float(np.median(secs[forwards // 3:]))
    layer = (med[4] - med[1]) / 3.0
    head = med[1] - layer
    per_forward = head + 48 * layer
    workers = cpu.lib.pkref_row_workers()
    return {"value": round(1.0 / per_forward, 4), "unit": "tokens/s", "cores": int(workers),
            "kind": "reference", "s_per_forward": round(per_forward, 4),
            "s_per_layer": round(layer, 5), "s_head": round(head, 5),
            "sample": f"reference runner on 1- and 4-layer models of the config-5 shape "
                      f"({prompt_len}-token prompt, median of the last {forwards - forwards // 3} "
                      f"of {forwards} greedy forwards each), extrapolated to 48 layers; "
                      f"row pool of {workers} workers; host nproc {os.cpu_count()}"}


def decode_cpu_full(prompt_len: int = 16, forwards: int = 8):
    """The reference Qwen3MoeRunner (oracle/_ref) on the full 48-layer
    config-5 model itself (a ~19 GB GGUF in /dev/shm, or /tmp when /dev/shm
    is too small), all experts cached after the prompt: seconds of each
    greedy forward (about 40 s on the GPU box's host).  None when the
    reference library is not built or no directory has room for the file;
    the decode leg then extrapolates from 1 and 4 layers."""
    import shutil

    import numpy as np

    import oracle
    from pokitlms_amd import gguf
    from pokitlms_amd import synth_model as SM
    if not oracle.available("reference"):
        return None
    cpu = oracle.Oracle("reference")
    m = SM.Qwen3MoeShape()
    need = sum(gguf.payload_bytes(g, dims) for _, dims, g, _ in SM.tensor_list(m))
    d = next((c for c in ("/dev/shm", "/tmp")
              if os.path.isdir(c) and shutil.disk_usage(c).free > need * 1.1 + (1 << 30)), None)
    if d is None:
        log(f"no directory with {need / 1e9:.1f} GB free for the 48-layer model file")
        return None
    path = os.path.join(d, f"pk_bench_decode_full_{os.getpid()}.gguf")
    step = [0]

    def progress(done, total):
        if done * 20 // total > step[0]:
            step[0] = done * 20 // total
            log(f"writing the 48-layer model: {done}/{total} tensors")

    try:
        SM.write_gguf(path, m, 1234, progress)
        log(f"model file {os.path.getsize(path) / 1e9:.2f} GB in {d}; running the reference runner")
        secs = cpu.qwen3moe_forward_times(path, SM.prompt_tokens(1234, prompt_len, m.vocab), forwards)
    finally:
        if os.path.exists(path):
            os.remove(path)
    steady = secs[forwards // 4:]
    per_forward = float(np.median(steady))
    workers = cpu.lib.pkref_row_workers()
    return {"value": round(1.0 / per_forward, 4), "unit": "tokens/s", "cores": int(workers),
            "kind": "reference", "s_per_forward": round(per_forward, 4),
            "forward_seconds": [round(float(t), 4) for t in secs],
            "sample": f"reference runner on the full 48-layer config-5 model ({prompt_len}-token "
                      f"prompt, median of the last {steady.size} of {forwards} greedy forwards); "
                      f"row pool of {workers} workers; host nproc {os.cpu_count()}"}


def divergence_report(ref, fast):
    """Where fast greedy tokens leave the golden ones: the golden logits' top-2
    gap against the fast logits' error at that step.  near_tie: the gap is
    within what the error can move (each of the two logits by up to the
    largest error, in opposite directions); otherwise the divergence is not
    reassociation noise."""
    import numpy as np
    t1, t2 = (int(i) for i in np.argsort(ref)[::-1][:2])
    gap = float(ref[t1] - ref[t2])
    err = np.abs(fast.astype(np.float64) - ref.astype(np.float64))
    return {"golden_top2": [t1, t2], "golden_gap": gap, "fast_argmax": int(np.argmax(fast)),
            "fast_max_abs_error": float(err.max()),
            "fast_pair_error": float(abs((fast[t1] - fast[t2]) - gap)),
            "fast_normwise": float(err.max() / np.abs(ref).max()),
            "near_tie": bool(gap <= 2.0 * float(err.max()))}


def decode_leg(torch, hip, with_cpu: bool):
    """Whole-model greedy decode: the seeded 48-layer
    30B-A3B-shape model generated in HBM, the golden 128-token prompt, 256
    greedy tokens.  Reference-order kernels (token parity with the CPU
    runner's golden tokens) and the bandwidth-optimised kernels."""
    import numpy as np

    from pokitlms_amd import synth_model as SM
    from pokitlms_amd.model import Qwen3MoeModel
    with np.load(os.path.join(ROOT, "tests", "golden", "model_golden.npz"),
                 allow_pickle=False) as z:
        seed, prompt, golden = int(z["full_seed"]), z["full_prompt"], z["full_tokens"]
        ref_decode_s = float(z["full_decode_seconds"]) if "full_decode_seconds" in z.files else None
    shape = SM.Qwen3MoeShape()
    n_new = len(golden)
    out = {"workload": "seeded 48-layer Qwen3-MoE 30B-A3B-shape model in HBM (Q4_K attention "
                       "and experts, Q6_K down and output head, F32 router/norms), 128-token "
                       "prompt, 256 greedy tokens",
           "weight_bytes_per_forward": decode_weight_bytes(shape)}
    # the fast kernels run first: where their tokens leave the golden ones, the
    # logits of that step are taken from both modes (the reference-order ones
    # are the CPU's, bit for bit) to tell a near-tie from a kernel error
    ctx, fast_logits = None, None
    for mode, ref in (("fast", False), ("reference_order", True)):
        with Qwen3MoeModel.synthetic(hip, shape, seed, reference_order=ref) as model:
            model.generate(prompt[:8], 4)  # warm-up: graph capture, first-touch
            tokens, _, st = model.generate(prompt, n_new)
            same = tokens == golden
            first_diff = -1 if same.all() else int(np.argmin(same))
            if not ref and first_diff >= 0:
                ctx = np.concatenate([prompt, golden[:first_diff]]).astype(np.uint32)
                fast_logits = model.generate(ctx, 1, want_logits=True)[1]
            ref_logits = model.generate(ctx, 1, want_logits=True)[1] if ref and ctx is not None else None
        dec_s = st["decode_ns"] / 1e9
        fwd_s = dec_s / st["decode_forwards"]
        out[mode] = {"forwards_per_s": round(st["decode_forwards"] / dec_s, 2),
                     "generated_tokens_per_s": round(n_new / dec_s, 2),
                     "ms_per_forward": round(fwd_s * 1e3, 3),
                     "prefill_ms": round(st["prefill_ns"] / 1e6, 1),
                     "weight_gbs": round(out["weight_bytes_per_forward"] / fwd_s / 1e9, 1),
                     "tokens_equal_golden": bool(same.all()), "first_mismatch": first_diff}
        if ref_logits is not None:
            out["fast"]["first_mismatch_logits"] = divergence_report(ref_logits, fast_logits)
        log(f"decode {mode}: {fwd_s * 1e3:.3f} ms/forward, first mismatch {first_diff}")
    out["token_parity"] = out["reference_order"]["tokens_equal_golden"]
    if ref_decode_s:
        out["golden_cpu_s_per_forward"] = round(ref_decode_s / (n_new - 1), 4)
    if with_cpu:
        log("decode cpu baseline (the reference runner on the full model) ...")
        cpu = decode_cpu_full()
        if cpu is None:
            cpu = decode_cpu_baseline()
        if cpu:
            cpu.update(cpu_info())
        out["cpu_baseline"] = cpu
        if cpu:
            # token parity holds in reference order only; the fast kernels'
            # tokens leave the reference's (see "fast"), so no speed-up is
            # claimed for them
            out["reference_order"]["speedup_vs_cpu"] = round(
                out["reference_order"]["forwards_per_s"] / cpu["value"], 1)
    out["fast"]["token_parity"] = False
    return out


def cpu_baseline(seconds: float):
    """The reference CPU MoE block (oracle/_ref, compiled from the reference's
    own sources) on one layer of the same shape; falls back to the C port."""
    import numpy as np

    import oracle
    from pokitlms_amd import synth as S
    kind = "reference" if oracle.available("reference") else "port"
    cpu = oracle.Oracle(kind)
    layer = S.moe_layer(seed=3)
    blk = cpu.moe(layer)
    g = S.rng(33)
    xs = S.normal_f32(g, 64 * 2048).reshape(64, 2048)
    blk.forward(xs[0])  # warm-up
    n, t0 = 0, time.perf_counter()
    times = []
    while True:
        t1 = time.perf_counter()
        blk.forward(xs[n % 64])
        times.append(time.perf_counter() - t1)
        n += 1
        if time.perf_counter() - t0 >= seconds and n >= 5:
            break
    med = float(np.median(times))
    cores = cpu.lib.pkref_row_workers() if kind == "reference" else 1
    return {
        **cpu_info(),
        "value": round(layer.routed_bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "cores": int(cores),
        "kind": kind,
        "ms_per_token": round(med * 1e3, 3),
        "sample": f"{n} single-token MoE-layer passes (config-3 shape, seed 3), median "
                  f"wall time; reference row pool of {cores} workers, router single-threaded; "
                  f"host nproc {os.cpu_count()}",
    }


TRACE_SLOTS = {"router": ("start", "inputs in", "done"),
               "gate_up": ("start", "ranked", "routes shared", "loads issued", "done"),
               "down": ("start", "loads issued", "dots done", "partials shared", "done")}


def timeline_leg(torch, hip, step_args, stream, steps: int = 30, reps: int = 7):
    """Per-phase times of one MoE-layer step from the kernels' own stamps
    (pk_hip_moe_decode_traced_async: the 100 MHz s_memrealtime counter read by
    every wave at fixed points).  A graph of `steps` traced steps (the timed
    run's layers and tokens) is replayed `reps` times; the trace then holds the
    last step, whose phases are given in microseconds after the first router
    wave's start: the 10th percentile, median and 90th percentile over the
    kernel's waves, pooled over the replays."""
    import numpy as np
    from pokitlms_amd import _abi
    dev = torch.device("cuda:0")
    trace = torch.zeros(_abi.TRACE_WORDS, dtype=torch.int64, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        cs = torch.cuda.current_stream().cuda_stream
        for i in range(steps):
            layer, x, y, ids, p = step_args(i)
            hip.moe_decode_traced_async(layer, x, y, ids, p, trace.data_ptr(), cs)
    pooled = {k: [[] for _ in v] for k, v in TRACE_SLOTS.items()}
    for _ in range(reps):
        trace.zero_()
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        t = trace.cpu().numpy().reshape(3, 8192, 8)
        t0 = t[0, :, 0][t[0, :, 0] > 0].min()
        for k, (name, slots) in enumerate(TRACE_SLOTS.items()):
            live = t[k, :, 0] > 0
            for j in range(len(slots)):
                pooled[name][j].extend(((t[k, live, j] - t0) / 100.0).tolist())
    out = {}
    for name, slots in TRACE_SLOTS.items():
        out[name] = {slot: [round(float(np.percentile(v, q)), 2) for q in (10, 50, 90)]
                     for slot, v in zip(slots, pooled[name])}
        out[name]["waves"] = len(pooled[name][0]) // reps
    return out


def timeline_markdown(tl) -> str:
    rows = ["| Kernel | Point | p10 µs | median µs | p90 µs |", "|---|---|---:|---:|---:|"]
    for name, slots in TRACE_SLOTS.items():
        for slot in slots:
            a, b, c = tl[name][slot]
            rows.append(f"| {name} ({tl[name]['waves']} waves) | {slot} | {a:.2f} | {b:.2f} | {c:.2f} |")
    return "\n".join(rows)


def flatten_summary(out, floors, matvec, decode):
    """The other configs' headline figures as flat scalar fields of the
    `roofline` and `cpu_baseline` objects (readers that keep only scalar
    fields of known objects still see them): config-1/2 matvec times and HBM
    fractions with their reference CPU times, the plain-read floors, and the
    config-5 decode's ms/forward, HBM fraction, token parity and CPU time."""
    rl, cb = out["roofline"], out["cpu_baseline"]
    rl["step_us"] = out["ms_per_step"] * 1e3
    if floors:
        for name, f in floors.items():
            rl[f"floor_{name}_us"] = f["us"]
            rl[f"floor_{name}_frac"] = f["frac"]
        rl["step_vs_floor"] = round(floors["step"]["us"] / rl["step_us"], 4)
    if matvec:
        for m in matvec:
            key = (f"c1" if m["config"] == "c1" else
                   "head" if m["config"] == "c5_head" else
                   f"c2_{m['type']}_{m['out']}x{m['in']}_b{m['batch']}")
            rl[f"{key}_us"] = m["us_graph"]
            rl[f"{key}_frac"] = round(m["gbs_graph"] / HBM_PEAK_GBS, 4)
            if cb is not None and "cpu_us" in m:
                cb[f"{key}_cpu_us"] = m["cpu_us"]
    if decode:
        ro = decode["reference_order"]
        rl["c5_ms_per_forward"] = ro["ms_per_forward"]
        rl["c5_hbm_frac"] = round(ro["weight_gbs"] / HBM_PEAK_GBS, 4)
        rl["c5_token_parity"] = bool(decode["token_parity"])
        rl["c5_fast_ms_per_forward"] = decode["fast"]["ms_per_forward"]
        c5cpu = decode.get("cpu_baseline")
        if cb is not None and c5cpu:
            cb["c5_s_per_forward"] = c5cpu["s_per_forward"]
            cb["c5_speedup"] = ro.get("speedup_vs_cpu")


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    if args.decode_cpu_full:
        print(json.dumps({"decode_cpu_full": decode_cpu_full()}), flush=True)
        return

    import numpy as np
    import torch

    from pokitlms_amd.backend import HipBackend

    dev = torch.device("cuda:0")
    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib << 18  # float32 elements
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 x {args.calibrate_copy_mib} MiB device copies")
        del src, dst
    hip = HipBackend(0)
    if args.matvec_only:
        print(json.dumps({"matvec": matvec_leg(torch, hip, torch.cuda.Stream(),
                                               args.matvec_reps)}), flush=True)
        hip.close()
        return
    log(f"building {args.layers} resident layers ...")
    layers = build_layers(torch, hip, args.layers, dev)
    step_bytes = layers[0].routed_bytes()
    assert step_bytes == 25_526_272, step_bytes
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    X = torch.randn(args.tokens, 2048, device=dev, generator=gen)
    Y = torch.empty(args.tokens, 2048, device=dev)
    IDS = torch.empty(args.tokens, 8, dtype=torch.int32, device=dev)
    P = torch.empty(args.tokens, 8, dtype=torch.float32, device=dev)

    stream = torch.cuda.Stream()
    torch.cuda.synchronize()

    def step_args(i):
        t = i % args.tokens
        return layers[i % args.layers], X[t].data_ptr(), Y[t].data_ptr(), IDS[t].data_ptr(), \
            P[t].data_ptr()

    def step(i, s):
        hip.moe_decode_async(*step_args(i), s)

    if args.timeline:
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                step(i, stream.cuda_stream)
        hip.sync(stream.cuda_stream)
        tl = timeline_leg(torch, hip, step_args, stream)
        print(timeline_markdown(tl), file=sys.stderr, flush=True)
        print(json.dumps({"timeline": tl}), flush=True)
        for l in layers:
            l.release()
        hip.close()
        return

    with torch.cuda.stream(stream):
        s = stream.cuda_stream
        for i in range(args.warmup):
            step(i, s)
        hip.sync(s)
        if not bool(torch.isfinite(Y).all()):
            raise RuntimeError("non-finite MoE output in warm-up")
        # eager reference for the graph check: the same `steps` steps, so every
        # output slot holds the result of the same final step
        for i in range(args.steps):
            step(i, s)
        hip.sync(s)
        y_eager, ids_eager = Y.clone(), IDS.clone()

        # eager timing (host launch bound; reported beside the graph figure)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n_eager = min(args.steps, 500)
        ev0.record(stream)
        for i in range(n_eager):
            step(i, s)
        ev1.record(stream)
        ev1.synchronize()
        eager_ms = ev0.elapsed_time(ev1) / n_eager

    chunk = min(args.graph_chunk, args.steps)
    if args.steps % chunk:
        chunk = args.steps
    graphs = []
    if not args.eager:
        for c in range(args.steps // chunk):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                cs = torch.cuda.current_stream().cuda_stream
                for i in range(c * chunk, (c + 1) * chunk):
                    step(i, cs)
            graphs.append(g)
        with torch.cuda.stream(stream):
            for g in graphs:  # untimed first replay: graph upload
                g.replay()
            hip.sync(stream.cuda_stream)
        # every replay must reproduce the eager result (first --tokens steps)
        ok_graph = bool(torch.equal(Y, y_eager) and torch.equal(IDS, ids_eager))

    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(stream)
        if args.eager:
            for i in range(args.steps):
                step(i, stream.cuda_stream)
        else:
            for g in graphs:
                g.replay()
        ev1.record(stream)
        ev1.synchronize()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gpu_ms = ev0.elapsed_time(ev1)
        hip.sync(stream.cuda_stream)
    graph_diag = None
    if not args.eager:
        ok_graph = ok_graph and bool(torch.equal(Y, y_eager) and torch.equal(IDS, ids_eager))
        bad_y = (Y != y_eager).any(dim=1)
        bad_i = (IDS != ids_eager).any(dim=1)
        graph_diag = {"slots_y_differ": int(bad_y.sum()), "slots_ids_differ": int(bad_i.sum()),
                      "max_abs_diff": float((Y - y_eager).abs().max())}
    ms_per_step = gpu_ms / args.steps
    value = step_bytes * args.steps / (gpu_ms / 1e3) / 1e9

    # per-kernel device time with HIP events on the launch stream
    hip.reset_stats()
    hip.set_kernel_timing(True)
    n_timed = 200
    with torch.cuda.stream(stream):
        for i in range(n_timed):
            step(i, stream.cuda_stream)
    hip.set_kernel_timing(False)
    st = hip.stats()
    kbytes = {
        # algorithmic bytes per launch: weights + activations in/out
        "k_router": 1_048_576 + 2048 * 4 + 8 * 8,
        "k_gate_up": 8 * 2 * 884_736 + 2048 * 4 + 8 * 768 * 4,
        "k_down": 8 * 1_290_240 + 8 * 768 * 4 + 2048 * 4,
    }
    kns = {"k_router": st["router_ns"] / n_timed, "k_gate_up": st["gate_up_ns"] / n_timed,
           "k_down": st["down_ns"] / n_timed}
    kernels = {k: {"avg_us": round(kns[k] / 1e3, 3), "bytes": kbytes[k],
                   "gbs": round(kbytes[k] / kns[k], 1) if kns[k] else None} for k in kns}
    dominant = max(kns, key=lambda k: kns[k])
    achieved = kbytes[dominant] / kns[dominant]  # B/ns == GB/s
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": profiled_traffic(dominant), "kernel": dominant,
                "avg_us": round(kns[dominant] / 1e3, 3), "algorithmic_bytes": kbytes[dominant]}

    # a spot parity check of the timed path against the CPU oracle
    parity = None
    try:
        import oracle
        from pokitlms_amd import synth as S
        layer = S.moe_layer(seed=3)
        h = hip.upload_moe_layer(layer)
        x = S.normal_f32(S.rng(33), 2048)
        y, ids, _ = hip.moe_decode(h, x)
        cy, cids, _ = oracle.Oracle("port").moe(layer).forward(x)
        parity = {"ids_equal": bool(np.array_equal(ids, cids)),
                  "normwise_rel": float(np.max(np.abs(y - cy)) / np.max(np.abs(cy)))}
        h.release()
    except Exception as e:  # reported, never fatal for the timing
        parity = {"error": str(e)}

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    prefill = None
    if not args.no_prefill:
        log("prefill leg ...")
        prefill = prefill_leg(torch, hip, layers[:4], stream, args.prefill_reps, not args.no_cpu)

    floors = None
    if not args.no_floor:
        log("read-floor leg ...")
        floors = floor_leg(torch, hip, stream)

    matvec = None
    if not args.no_matvec:
        log("matvec leg ...")
        matvec = matvec_leg(torch, hip, stream, args.matvec_reps, with_cpu=not args.no_cpu)

    decode = None
    if not args.no_decode:
        log("whole-model decode leg ...")
        for l in layers:
            l.release()
        layers = []
        decode = decode_leg(torch, hip, not args.no_cpu)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init weights generated on the GPU, x ~ N(0,1))",
        "config": {
            "workload": "single-token Qwen3-MoE layer (BASELINE configs[2]): hidden 2048, "
                        "128 experts, top-8 renormalised, F32 router, gate/up Q4_K 768x2048, "
                        "down Q6_K 2048x768",
            "layers_rotated": args.layers, "tokens_rotated": args.tokens,
            "bytes_per_step": step_bytes,
            "timing": "eager" if args.eager else f"HIP graph replay, {chunk} steps per graph",
            "launches_per_step": 3,
        },
        "pct_of_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "eager_ms_per_step": round(eager_ms, 5),
        "wall_s": round(wall, 4),
        "roofline": roofline,
        "kernels": kernels,
        "router_fallbacks_per_1k": round(1000.0 * st["router_fallbacks"] / n_timed, 2),
        "graph_matches_eager": None if args.eager else ok_graph,
        "graph_check": graph_diag,
        "parity": parity,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "matvec": matvec,
        "decode": decode,
    }
    if cpu:
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    out["floors"] = floors
    flatten_summary(out, floors, matvec, decode)
    print(json.dumps(out), flush=True)
    for l in layers:
        l.release()
    hip.close()


if __name__ == "__main__":
    main()
