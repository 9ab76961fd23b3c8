#!/usr/bin/env python3
"""Sampler benchmark: sampled rows/s and HBM roofline on one MI355X.

One step = one engine step's sampling: a single ``pbs_sample`` launch over all rows of
the ``mixed256_llama3_bf16`` workload (bf16 logits [256, 128256], mixed temperature /
top-k / top-p per row). Inputs are resident in HBM before timing; the step rotates over
several copies of the logits (> 256 MB in total) so the 256 MB Infinity Cache cannot
serve a step from the previous one. Per-row parameters and uniforms live on the device.
The K timed steps are one replay of a HIP graph holding the K launches (``value``,
``ms_per_step``); HIP events on the launch stream around that replay give the kernel's
average duration (``us_per_step_kernel``, the roofline's time base, the figure the
rocprofv3 kernel trace reports). Each launch is also timed on its own with an event pair
(``us_per_launch_events``, which also spans the launch's dispatch), and the Python
``sample()`` surface per step is reported as ``us_per_step_python`` (256 seeded
generators) with its split into uniforms, packing and launch + copy back + sync for one
shared generator and for 256 seeded ones, and for the same call replayed from a HIP graph
(``python_surface``).

``--workload engine_step_smollm2`` instead runs the end-to-end engine step
(pagedbatch_amd/engine_step.py) and reports decode tokens/s and the sampler's share.

Prints one JSON line (rank 0): the workload's metric with its value and unit, plus a
``roofline`` object for the sampling kernel and a ``cpu_baseline`` object (the op-for-op
CPU restatement of pagedbatch/sampling.py timed on this host in the same run).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, 8 TB/s
METRIC = "sampled rows/s + HBM GB/s (% peak), bf16 logits 256×128256 mixed top-k/p"


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="mixed256_llama3_bf16",
                    choices=["mixed256_llama3_bf16", "greedy512_quantized", "nucleus1024_qwen_fp32",
                             "steps8_smollm_mixed", "engine_step_smollm2", "lm_head_smollm2"])
    ap.add_argument("--copies", type=int, default=0, help="logits copies to rotate over (default: > 256 MB)")
    ap.add_argument("--cpu-steps", type=int, default=5, help="CPU baseline steps (median)")
    ap.add_argument("--cpu-rows", type=int, default=0, help="CPU baseline rows per step (0: all)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-parity", action="store_true", help="skip the token check against the oracle")
    ap.add_argument("--copy-only", action="store_true",
                    help="time a plain device copy of the workload's logits bytes instead of the sampler "
                         "(the reference kernel for calibrating HBM byte counters)")
    return ap.parse_args()


def copy_only(args, w, torch):
    """Plain copy of the same byte count as one step's logits (dst <- src, rotating buffers)."""
    nbytes = w.rows * w.vocab * w.logits.element_size()
    copies = args.copies or max(2, -(-300_000_000 // nbytes))
    src = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1) for _ in range(copies)]
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for i in range(args.warmup):
        dst.copy_(src[i % copies])
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record()
    for i in range(args.steps):
        dst.copy_(src[i % copies])
    g1.record()
    torch.cuda.synchronize()
    ms = g0.elapsed_time(g1) / args.steps
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "steps": args.steps,
                      "ms_per_copy": round(ms, 5), "GBps_read_plus_write": round(2 * nbytes / ms / 1e6, 1)}),
          flush=True)


def cpu_baseline(w, steps: int, rows: int):
    """Time the op-for-op CPU restatement of sampling.py (engine.py:133-139 row loop).

    Runs with every core the process may use (the reported figure) and again with one
    thread (reported beside it), median over ``steps`` steps each.
    """
    import torch

    from oracle.reference_ops import engine_step_ops

    cores = len(os.sched_getaffinity(0))
    n = rows or w.rows
    logits = w.logits[:n].contiguous()
    params = [(w.temperature[i], w.top_k[i], w.top_p[i]) for i in range(n)]

    def run(threads, nsteps):
        torch.set_num_threads(threads)
        times = []
        for s in range(nsteps):
            gens = [torch.Generator().manual_seed(1000 * s + i) for i in range(n)]
            t0 = time.perf_counter()
            engine_step_ops(logits, params, gens)
            times.append(time.perf_counter() - t0)
        return statistics.median(times)

    med = run(cores, steps)
    med1 = run(1, max(1, min(steps, 3)))
    torch.set_num_threads(cores)
    return {
        "value": round(n / med, 3),
        "unit": "rows/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n} of {w.rows} rows of {w.name}, median of {steps} steps "
                  f"({med * 1e3:.1f} ms/step, {med / n * 1e3:.2f} ms/row), torch {torch.__version__} CPU; "
                  f"1 thread: {n / med1:.3f} rows/s ({med1 * 1e3:.1f} ms/step)",
        "value_1_thread": round(n / med1, 3),
    }


def source_sha() -> str:
    """sha256 (first 16 hex digits) of the sampler kernel source the library is built from."""
    import hashlib

    with open(os.path.join(ROOT, "pagedbatch_amd", "csrc", "pbsample.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def committed_traffic(workload: str):
    """HBM bytes per launch from the committed counter profile
    (profiles/traffic_<workload>.json, written from two rocprofv3 --pmc runs), reported only
    when that profile was measured on the kernel source this library is built from."""
    tpath = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(tpath):
        return None, "no committed counter profile for this workload"
    with open(tpath) as f:
        prof = json.load(f)
    sha = source_sha()
    if prof.get("source_sha") != sha:
        return None, (f"profiles/traffic_{workload}.json was measured on kernel source "
                      f"{prof.get('source_sha')}, this build is {sha}: not reported")
    return prof.get("hbm_bytes_per_launch"), (f"profiles/traffic_{workload}.json (rocprofv3 FETCH_SIZE + "
                                               f"WRITE_SIZE, calibrated on a copy kernel; kernel source {sha})")


def python_surface(w, bufs, copies, rows):
    """The whole Python ``sample()`` surface per engine step, median of 20 calls, split into
    the uniforms (one torch.rand per run of rows sharing a generator), packing the
    parameters into the pinned staging block, and the launch plus the copy back and the
    synchronisation; once with one shared generator (the engine's, engine.py:58) and once
    with a seeded generator per row (every request seeded, engine.py:84)."""
    import torch

    from pagedbatch_amd import SamplingParams
    from pagedbatch_amd.sampling import _sample

    sp = [SamplingParams(temperature=w.temperature[i], top_k=w.top_k[i], top_p=w.top_p[i]) for i in range(rows)]
    out = {}
    for name in ("shared_generator", "seeded_generators"):
        shared = torch.Generator().manual_seed(0)
        gens = [shared] * rows if name == "shared_generator" else [torch.Generator().manual_seed(i)
                                                                 for i in range(rows)]
        for i in range(3):
            _sample(bufs[i % copies], sp, gens, None)
        parts = {"uniforms_us": [], "pack_us": [], "launch_sync_us": [], "total_us": []}
        for i in range(20):
            tm = {}
            t0 = time.perf_counter()
            _sample(bufs[i % copies], sp, gens, None, timing=tm)
            t1 = time.perf_counter()
            parts["uniforms_us"].append(tm["uniforms"] - tm["start"])
            parts["pack_us"].append(tm["pack"] - tm["uniforms"])
            parts["launch_sync_us"].append(tm["launch_sync"] - tm["pack"])
            parts["total_us"].append(t1 - t0)
        out[name] = {k: round(statistics.median(v) * 1e6, 1) for k, v in parts.items()}
    # the same call captured in a HIP graph (sampling.SamplingGraph on one fixed logits
    # buffer): per step only the uniforms, the replay and one synchronisation
    from pagedbatch_amd import SamplingGraph

    for name in ("shared_generator_graph", "seeded_generators_graph"):
        shared = torch.Generator().manual_seed(0)
        gens = [shared] * rows if name.startswith("shared") else [torch.Generator().manual_seed(i)
                                                                  for i in range(rows)]
        sg = SamplingGraph(bufs[0], sp)
        for i in range(3):
            sg(gens)
        ts = []
        for i in range(20):
            t0 = time.perf_counter()
            sg(gens)
            ts.append(time.perf_counter() - t0)
        out[name] = {"total_us": round(statistics.median(ts) * 1e6, 1)}
    return out


def engine_sampler_kernel_us(cap) -> float:
    """The sampling kernel alone on one decode step's logits (bf16 [64, 49152], the step's
    own parameters and uniforms): mean of 50 back-to-back launches between HIP events on
    the launch stream."""
    import torch

    from pagedbatch_amd import _lib
    from pagedbatch_amd.sampling import _TORCH_DTYPE

    dev = cap.logits.device
    lib = _lib.load()
    rows, vocab = cap.logits.shape
    T = torch.tensor(cap.temperature, dtype=torch.float32, device=dev)
    K = torch.tensor([k if 0 < k < vocab else 0 for k in cap.top_k], dtype=torch.int32, device=dev)
    P = torch.tensor(cap.top_p, dtype=torch.float32, device=dev)
    U = torch.tensor(cap.uniform, dtype=torch.float32, device=dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def launch():
        rc = lib.pbs_sample(cap.logits.data_ptr(), _TORCH_DTYPE[cap.logits.dtype], rows, rows, vocab, vocab, None,
                            T.data_ptr(), K.data_ptr(), P.data_ptr(), U.data_ptr(), tok.data_ptr(), st.data_ptr(),
                            None, 0, stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(_lib.last_error(lib))

    for _ in range(5):
        launch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(50):
        launch()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    assert tok.cpu().tolist() == cap.tokens
    return round(e0.elapsed_time(e1) * 1e3 / 50, 3)


def lm_head_bench(args):
    """The fused lm_head + greedy kernel at the smollm2-135m head (bf16 hidden [64, 576],
    weight [49152, 576]; pagedbatch/model.py:283 then sampling.py:12-13) against the unfused
    path (torch's bf16 Linear, then pbs_argmax over the logits it wrote). Weights rotate
    over 5 copies (283 MB) so HBM, not the Infinity Cache, serves them. Kernel times are
    HIP events around 100 back-to-back launches on the launch stream."""
    import torch
    import torch.nn.functional as F

    from pagedbatch_amd import _lib
    from pagedbatch_amd.lm_head import lm_head_argmax

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    rows, hdim, vocab = 64, 576, 49152
    g = torch.Generator().manual_seed(0)
    hidden = torch.randn(rows, hdim, generator=g).to(torch.bfloat16).to(dev)
    w0 = (torch.randn(vocab, hdim, generator=g) * 0.02).to(torch.bfloat16)
    copies = 5
    ws = [w0.to(dev) for _ in range(copies)]
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)

    def timed(fn, n=100):
        for i in range(10):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(n):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    def unfused(i):
        logits = F.linear(hidden, ws[i % copies])
        rc = lib.pbs_argmax(logits.data_ptr(), _lib.DTYPE_BF16, rows, rows, vocab, vocab, None, tok.data_ptr(),
                            st.data_ptr(), stream.cuda_stream)
        assert rc == 0

    us_fused = timed(lambda i: lm_head_argmax(hidden, ws[i % copies]))
    us_fused_nologits = timed(lambda i: lm_head_argmax(hidden, ws[i % copies], want_logits=False))
    us_linear = timed(lambda i: F.linear(hidden, ws[i % copies]))
    us_unfused = timed(unfused)
    # parity of the measured kernels: the fused tokens against the argmax of their own
    # logits and against the unfused path's tokens where torch's logits agree
    logits, t_f = lm_head_argmax(hidden, ws[0])
    unfused(0)
    torch.cuda.synchronize()
    same_logits = (logits == F.linear(hidden, ws[0])).float().mean().item()
    agree = (t_f == tok).float().mean().item()
    wbytes = vocab * hdim * 2
    traffic = wbytes + rows * hdim * 2 + rows * vocab * 2
    flops = 2.0 * rows * hdim * vocab
    out = {
        "metric": "lm_head + greedy per decode step (us), bf16 [64, 576] x [49152, 576]",
        "value": round(us_fused, 3),
        "unit": "us",
        "higher_is_better": False,
        "n_gpus": 1,
        "dtype": "bf16 (fp32 accumulation)",
        "data": "synthetic (random hidden and weights, seed 0)",
        "config": {"workload": "lm_head_smollm2", "rows": rows, "hidden": hdim, "vocab": vocab,
                   "weight_copies_rotated": copies},
        "us_fused_with_logits": round(us_fused, 3),
        "us_fused_greedy_only": round(us_fused_nologits, 3),
        "us_torch_linear": round(us_linear, 3),
        "us_torch_linear_then_pbs_argmax": round(us_unfused, 3),
        "roofline": {"bound": "hbm", "achieved": round(traffic / us_fused / 1e3, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(traffic / us_fused / 1e3 / HBM_PEAK_GBPS, 4),
                     "algorithmic_bytes_per_launch": traffic,
                     "mfma_tflops": round(flops / us_fused / 1e6, 1), "mfma_peak_tflops": 2500.0},
        "roofline_greedy_only": {"achieved": round((wbytes + rows * hdim * 2) / us_fused_nologits / 1e3, 1),
                                 "unit": "GB/s"},
        "parity": {"logits_equal_to_torch_linear": round(same_logits, 6), "tokens_equal_to_unfused": round(agree, 4)},
    }
    print(json.dumps(out), flush=True)


def engine_step(args):
    """The end-to-end engine step (smollm2-135m-random, 64 requests x 128 prompt + 128
    output tokens, half greedy, half top-k=50 / top-p=0.9): decode throughput (`value`:
    the decode forward replayed from a HIP graph with the paged-attention decode kernel,
    batched sampling) and the sampler's share of the step, also with the forward launched
    op by op, with one sampling call per row (torch attention) and with the fused lm_head."""
    import torch

    from pagedbatch_amd import engine_step as es

    shape = es.ModelShape()
    kw = dict(num_seqs=64, prompt_len=128, output_len=128, block_size=16, device="cuda")
    print("[bench] engine step: warm-up", file=sys.stderr, flush=True)
    es.run(shape, **{**kw, "output_len": 4})
    print("[bench] engine step: batched sampling", file=sys.stderr, flush=True)
    tb, out_b = es.run(shape, **kw)
    print("[bench] engine step: one sampling call per row", file=sys.stderr, flush=True)
    tr, out_r = es.run(shape, **kw, per_row=True)
    same = out_b == out_r
    print("[bench] engine step: batched sampling, paged-attention decode kernel", file=sys.stderr, flush=True)
    tf, out_f = es.run(shape, **kw, fused_decode=True, capture_steps=(kw["output_len"] - 1,))
    sampler_kernel_us = engine_sampler_kernel_us(tf.captures[0])
    print("[bench] engine step: fused lm_head + greedy, paged-attention decode kernel", file=sys.stderr, flush=True)
    th, out_h = es.run(shape, **kw, fused_decode=True, fused_head=True)
    print("[bench] engine step: decode forward replayed from a HIP graph, paged-attention decode kernel",
          file=sys.stderr, flush=True)
    tg, out_g = es.run(shape, **kw, fused_decode=True, graph=True)
    agree_head = sum(a == b for x, y in zip(out_f, out_h) for a, b in zip(x, y)) / sum(len(x) for x in out_f)
    # the fused attention rounds differently in the last fp32 bits, which the bf16 o_proj
    # input can turn into different tokens later in a sequence: report the agreement
    agree = sum(a == b for x, y in zip(out_b, out_f) for a, b in zip(x, y)) / sum(len(x) for x in out_b)

    def split(t):
        fwd, smp = t.forward_s[1:], t.sample_s[1:]  # decode steps (step 0 is the prefill)
        n = len(fwd)
        return {"decode_steps": n, "forward_ms": round(1e3 * sum(fwd) / n, 4),
                "sample_ms": round(1e3 * sum(smp) / n, 4),
                "sample_share": round(sum(smp) / (sum(fwd) + sum(smp)), 4),
                "prefill_forward_ms": round(1e3 * t.forward_s[0], 3), "prefill_sample_ms": round(1e3 * t.sample_s[0], 4)}

    b, r, f, hd, gr = split(tb), split(tr), split(tf), split(th), split(tg)
    # the graph replays the eager fused step's kernels: the same tokens, or the graph is wrong
    same_graph = out_g == out_f
    step_ms = gr["forward_ms"] + gr["sample_ms"]
    # the batched call runs the stop check (engine.py:173-182) on the device after the
    # sampler and brings the reasons back with the tokens: every request ends on "length"
    # at its 128th output, none before
    assert tb.reasons[-1] == ["length"] * 64 and all(x is None for rs in tb.reasons[:-1] for x in rs)
    line = {
        "metric": "engine decode tokens/s (smollm2-135m-random bf16, 64 requests, 128 prompt + 128 output tokens)",
        "value": round(64 / (step_ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": b["decode_steps"],
        "warmup": 1, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random weights, random prompt ids)",
        "config": {"workload": "engine_step_smollm2", "requests": 64, "prompt_len": 128, "output_len": 128,
                   "block_size": 16, "mix": "half greedy, half top_k=50 top_p=0.9 T=1.0",
                   "decode_attention": "paged-attention kernel (pba_decode_attention)",
                   "decode_forward": "HIP graph replay (engine_step.DecodeGraph)"},
        "graph_decode": {**gr, "same_tokens_as_eager": same_graph},
        "fused_decode_attention": f, "batched_sampling": b, "per_row_sampling": r,
        "fused_lm_head": {**hd, "note": "forward ends at the final hidden state; sample_ms includes the lm_head "
                                        "GEMM (pbs_lm_head_argmax) and the stochastic rows' sampling",
                          "ms_per_step": round(hd["forward_ms"] + hd["sample_ms"], 4),
                          "token_agreement_vs_torch_head": round(agree_head, 4)},
        "same_tokens_batched_vs_per_row": same, "token_agreement_fused_vs_torch_attention": round(agree, 4),
        "stop_check": "on the device after the sampler, reasons in the tokens' copy back (in sample_ms)",
        "sampler_kernel_us": sampler_kernel_us,
        "torch": torch.__version__,
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build samples on a single device and has no "
              f"multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    if args.workload == "engine_step_smollm2":
        engine_step(args)
        return
    if args.workload == "lm_head_smollm2":
        lm_head_bench(args)
        return

    import numpy as np
    import torch

    from pagedbatch_amd import _lib, workloads
    from pagedbatch_amd.sampling import _TORCH_DTYPE

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lib = _lib.load()
    print(f"[bench] building workload {args.workload}", file=sys.stderr, flush=True)
    w = workloads.WORKLOADS[args.workload]()
    if args.copy_only:
        copy_only(args, w, torch)
        return
    rows, vocab = w.rows, w.vocab
    elt = w.logits.element_size()
    alg_bytes = rows * vocab * elt
    copies = args.copies or max(2, -(-300_000_000 // alg_bytes))
    bufs = [w.logits.to(dev) for _ in range(copies)]
    T = torch.tensor(w.temperature, dtype=torch.float32, device=dev)
    K = torch.tensor([k if 0 < k < vocab else 0 for k in w.top_k], dtype=torch.int32, device=dev)
    P = torch.tensor(w.top_p, dtype=torch.float32, device=dev)
    U = torch.tensor(w.uniform, dtype=torch.float32, device=dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    st = torch.empty(rows, dtype=torch.int32, device=dev)
    dcode = _TORCH_DTYPE[w.logits.dtype]
    stream = torch.cuda.current_stream(dev)

    # a step whose rows are all greedy goes to the argmax kernel, as sample() routes it
    greedy = all(t == 0 for t in w.temperature)
    entry = "pbs_argmax" if greedy else "pbs_sample"

    def launch(i):
        x = bufs[i % copies]
        sp = torch.cuda.current_stream(dev).cuda_stream  # the capture stream inside a graph capture
        if greedy:
            rc = lib.pbs_argmax(x.data_ptr(), dcode, rows, rows, vocab, vocab, None, tok.data_ptr(), st.data_ptr(),
                                sp)
        else:
            rc = lib.pbs_sample(x.data_ptr(), dcode, rows, rows, vocab, vocab, None, T.data_ptr(), K.data_ptr(),
                                P.data_ptr(), U.data_ptr(), tok.data_ptr(), st.data_ptr(), None, 0, sp)
        if rc != 0:
            raise RuntimeError(f"{entry} failed: {_lib.last_error(lib)}")

    print(f"[bench] warmup {args.warmup}", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()

    # (1) per-launch kernel durations: HIP events around each launch, on the launch stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    print(f"[bench] per-launch timing, {args.steps} launches", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(stream)
        launch(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    per_launch_ms = [a.elapsed_time(b) for a, b in ev]
    kern_ms = statistics.mean(per_launch_ms)

    # (2) whole-job throughput: the K steps captured once in a HIP graph and replayed, so
    # the host's per-launch cost does not starve the GPU (an engine issues the sampler
    # behind the model's forward pass; us_per_step_python reports the Python surface)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(args.steps):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    print(f"[bench] timing {args.steps} steps (one graph replay)", file=sys.stderr, flush=True)
    g0 = torch.cuda.Event(enable_timing=True)
    g1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g0.record(stream)
    graph.replay()
    g1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_total_ms = g0.elapsed_time(g1)
    step_ms = max(wall * 1e3, gpu_total_ms) / args.steps
    value = rows / (step_ms / 1e3)
    # the roofline uses the kernel's average duration over the replayed launches (HIP events
    # on the launch stream around the timed replay: back-to-back launches, so this is the
    # kernel time the rocprofv3 trace reports); the per-launch event pairs above also span
    # each launch's dispatch and are reported beside it
    replay_kern_ms = gpu_total_ms / args.steps
    achieved = alg_bytes / (replay_kern_ms / 1e3) / 1e9

    status = st.cpu().numpy()
    tokens = tok.cpu().numpy()
    parity = None
    if not args.no_parity:
        from oracle import oracle
        from oracle.compare import compare_rows

        n = min(rows, 64)
        raw = w.logits[:n]
        raw = raw.view(torch.int16).numpy().view(np.uint16) if raw.dtype == torch.bfloat16 else raw.numpy()
        dt = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}[w.logits.dtype]
        refs = oracle.sample_batch(raw, dt, w.temperature[:n], w.top_k[:n], w.top_p[:n], w.uniform[:n])
        rep = compare_rows(tokens[:n], status[:n], refs, [t == 0 for t in w.temperature[:n]], top_p=w.top_p[:n],
                           uniform=w.uniform[:n])
        parity = {"rows": n, "ok": rep.ok(), "tokens_checked": rep.checked_tokens,
                  "tokens_in_band_checked_to_band_bar": rep.exempt_tokens}

    traffic, traffic_note = committed_traffic(args.workload)
    surface = python_surface(w, bufs, copies, rows)

    cpu = None
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(w, args.cpu_steps, args.cpu_rows)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "us_per_step_kernel": round(replay_kern_ms * 1e3, 3),
        "us_per_launch_events": round(kern_ms * 1e3, 3),
        "ms_per_step_eager_launches": round(eager_ms, 5),
        "us_per_step_python": surface["seeded_generators"]["total_us"],
        "python_surface": surface,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[w.logits.dtype],
        "data": "synthetic (seeded logits recipe, see pagedbatch_amd/workloads.py)",
        "config": {"workload": w.name, "rows": rows, "vocab": vocab, "logits_dtype": str(w.logits.dtype),
                   "buffers_rotated": copies, "parallelism": "single GPU"},
        "entry_point": entry,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_note, "algorithmic_bytes_per_launch": alg_bytes},
        "cpu_baseline": cpu,
        "speedup_vs_cpu": round(value / cpu["value"], 1) if cpu else None,
        "parity": parity,
        "row_status_ok": bool((status == 0).all()),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
