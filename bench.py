"""Benchmark of the MI355X MoE feed-forward path (DeepSeek-V2-Lite MoE layer).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode_t1] [--no-cpu]
    python bench.py --workload stack      # the 27-layer FFN stack at T=1 and T=4096
    python bench.py --workload load       # SafeTensors shards of 4 layers into HBM
    python bench.py --workload head       # final norm + LM head + greedy token, T=1
    python bench.py --workload attention  # one MLA attention layer: decode near 512 / 4K cache tokens, prefill T=512
    python bench.py --workload decoder    # 27 layers of attention + FFN: prefill of 512 tokens, then decode
    python bench.py --workload decode_t1_v2  # DeepSeek-V2's full MoE layer (160 experts, hidden 5120) at T=1

A step is one MoE-layer forward (router, permutation, routed + shared SwiGLU
experts, combine) over one batch of T synthetic tokens whose inputs are already
resident in HBM.  The headline workload is decode at T=1; it rotates through 8
independently seeded layers (1.15 GB each) so the 139 MB active set of a step
cannot be served from the 256 MB Infinity Cache.  The T=2048 skewed prefill
workload is measured in the same run and reported under "t2048".

Prints ONE JSON line (rank 0) with the throughput, the dominant kernel's
roofline fraction measured with HIP events on the library's stream, and
LiteMind's own CPU path (its kernels compiled from its sources) timed on a
bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/sec at T=1 and T=2048; % HBM BW (T=1) / % bf16 MFMA (T=2048)"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2516.6  # dense bf16/fp16 MFMA, 256 CU x 2.4 GHz x 4096 flop/clk/CU
PEAK_CLOCK_MHZ = 2400.0    # the engine clock that peak assumes

EXPERT_BYTES = 3 * 1408 * 2048 * 2          # 17,301,504
GATEUP_EXPERT_BYTES = 2 * 1408 * 2048 * 2   # 11,534,336
DOWN_EXPERT_BYTES = 1408 * 2048 * 2         # 5,767,168
SHARED_BYTES = 3 * 2816 * 2048 * 2          # 34,603,008
ROUTER_BYTES = 64 * 2048 * 4                # 524,288

# HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes over
# this benchmark, scaled by the counters' readings for a conversion kernel of
# known size (profiles/decode_fused_kernel_decode_t1_hbm_traffic.md and
# profiles/mfma_grouped_kernel_prefill_t2048_skewed.md).
MEASURED_TRAFFIC = {("decode_t1", "decode_fused_kernel"): 142_380_838,
                    ("prefill_t2048_skewed", "gate_up"): 1_261_440_220,
                    ("prefill_t2048_skewed", "down"): 705_484_080}


class ClockSampler:
    """The graphics clock while timed steps run: amdsmi's GPU metrics
    (current_gfxclks, MHz per XCD, averaged over the XCDs) polled every 0.5 ms
    from a thread.  summary() is None where amdsmi cannot read them."""

    def __init__(self):
        import threading
        self.samples, self.stop, self.thread, self.handle = [], threading.Event(), None, None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self.amdsmi = amdsmi
            self.handle = amdsmi.amdsmi_get_processor_handles()[0]
            self._read()
        except Exception as e:  # no metrics on this host: report none
            log(f"clock sampler unavailable: {e}")
            self.handle = None

    def _read(self):
        m = self.amdsmi.amdsmi_get_gpu_metrics_info(self.handle)
        xcd = [v for v in (m.get("current_gfxclks") or []) if isinstance(v, (int, float)) and v > 0]
        if xcd:
            return float(np.mean(xcd))
        v = m.get("current_gfxclk")
        return float(v) if isinstance(v, (int, float)) and v > 0 else None

    def _run(self):
        while not self.stop.is_set():
            try:
                v = self._read()
                if v is not None:
                    self.samples.append(v)
            except Exception:
                pass
            time.sleep(0.0005)

    def __enter__(self):
        import threading
        if self.handle is not None:
            self.stop.clear()
            self.thread = threading.Thread(target=self._run, daemon=True)
            self.thread.start()
        return self

    def __exit__(self, *exc):
        if self.thread is not None:
            self.stop.set()
            self.thread.join()
            self.thread = None

    def summary(self) -> dict | None:
        if not self.samples:
            return None
        a = np.array(self.samples)
        return {"mhz": round(float(np.median(a)), 1), "min_mhz": round(float(a.min()), 1),
                "max_mhz": round(float(a.max()), 1), "samples": int(a.size),
                "source": "amdsmi gpu metrics current_gfxclks (mean over XCDs), median over the timed steps"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic(tokens: int, distinct_experts: int, act_bytes: int = 4) -> dict:
    """Bytes and flops of one MoE layer step (weights read once, activations in/out).
    act_bytes: width of the expert kernels' input and intermediate activations
    (fp32 on the GEMV path, fp16 panels on the MFMA path)."""
    T, U = tokens, distinct_experts
    H, I, S, K = 2048, 1408, 2816, 6
    layer_bytes = U * EXPERT_BYTES + SHARED_BYTES + ROUTER_BYTES + T * H * 4 * 2
    gate_up_bytes = U * GATEUP_EXPERT_BYTES + 2 * S * H * 2 + T * H * act_bytes + (T * K * I + T * S) * act_bytes
    down_bytes = U * DOWN_EXPERT_BYTES + S * H * 2 + (T * K * I + T * S) * act_bytes + (T * K + T) * H * 4
    flops_assign = 6 * H * I
    layer_flops = T * K * flops_assign + T * 6 * H * S + T * 2 * 64 * H
    gate_up_flops = T * K * 4 * H * I + T * 4 * H * S
    down_flops = T * K * 2 * H * I + T * 2 * H * S
    return dict(layer_bytes=layer_bytes, gate_up_bytes=gate_up_bytes, down_bytes=down_bytes,
                layer_flops=layer_flops, gate_up_flops=gate_up_flops, down_flops=down_flops)


def run_gpu(workload_name: str, steps: int, warmup: int, rotate: int, path: int):
    from litemind_amd import STAGES, Context
    from litemind_amd import workload as wl

    w = wl.WORKLOADS[workload_name]
    dims = wl.V2_LITE
    T = w.tokens
    log(f"{workload_name}: generating {rotate} layer(s) and uploading")
    ctx = Context(dims.moe_config(num_layers=rotate))
    layers = []
    for l in range(rotate):
        L = wl.moe_layer(wl.MASTER_SEED + l, 0, dims, router_scale=w.router_scale)
        wl.upload_moe_layer(ctx, l, L)
        layers.append(L)
    x = wl.tokens(wl.MASTER_SEED + 7, T, dims.hidden)
    bias = wl.skew_bias() if w.skewed else None
    dx = ctx.to_device(x)
    dy = ctx.empty((T, dims.hidden))
    didx = ctx.empty((rotate, T, dims.top_k), np.int32)
    dw = ctx.empty((rotate, T, dims.top_k))
    db = ctx.to_device(bias) if bias is not None else None
    idx_stride = T * dims.top_k * 4

    def step(i):
        l = i % rotate
        ctx.moe_forward(l, dx, T, dy, bias=db, idx=didx.ptr + l * idx_stride, w=dw.ptr + l * idx_stride, path=path)

    log(f"{workload_name}: warmup {warmup}")
    for i in range(warmup):
        step(i)
    ctx.synchronize()
    start_ev, stop_ev = ctx.event(), ctx.event()
    ctx.synchronize()
    clock = ClockSampler()
    with clock:
        t0 = time.perf_counter()
        ctx.record(start_ev)
        for i in range(steps):
            step(i)
        ctx.record(stop_ev)
        ctx.synchronize()
        wall = time.perf_counter() - t0
    gpu_ms = ctx.elapsed_ms(start_ev, stop_ev)
    log(f"{workload_name}: {steps} steps wall {wall * 1e3:.3f} ms, events {gpu_ms:.3f} ms")

    # Per-stage durations with HIP events between the stages, in a second timed
    # pass (a single token is one kernel per step: nothing to split; that pass
    # then only carries the clock probe).  The core clock of that pass comes
    # from the in-kernel probe: one wave on a second stream reads the core
    # clock counter and the 100 MHz real-time counter every 20 us.
    stages = {}
    probe = None
    probe_s = min(2.0, gpu_ms * 1e-3 * 1.2 + 1e-3)
    if T > 1:
        ctx.stage_timing(True)
    ctx.clock_probe_start(probe_s)
    with clock:
        for i in range(steps):
            step(i)
        ctx.synchronize()
    probe = ctx.clock_probe_finish()
    probe["source"] = ("s_memtime cycles per s_memrealtime tick (100 MHz), 20 us intervals, one wave on a second "
                       "stream during a second pass of the same steps; median")
    if T > 1:
        stages = ctx.stage_times()
        ctx.stage_timing(False)

    idx_all = didx.download()
    distinct = [len(np.unique(idx_all[l])) for l in range(min(rotate, steps))]
    U = float(np.mean(distinct))
    ctx.close()
    return dict(T=T, wall_s=wall, gpu_ms=gpu_ms, steps=steps, stages=stages, distinct=U, layers=layers, x=x,
                bias=bias, workload=workload_name, clock=probe if probe and probe["intervals"] else clock.summary(),
                clock_amdsmi=clock.summary())


def run_stack(steps_t1: int, steps_big: int, big_tokens: int, moe_layers: int) -> dict:
    """The full FFN stack: dense layer 0, then `moe_layers` MoE layers (independent
    seeds), chained through RMSNorm (weights 1) and the residual add, resident in
    HBM.  A step is one pass of T tokens through every layer.  (Parity of the
    chain is tests/test_gpu_stack.py.)"""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    n = 1 + moe_layers
    log(f"stack: generating and uploading dense + {moe_layers} MoE layers")
    ctx = Context(dims.moe_config(num_layers=n))
    gate, up, down = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
    ctx.upload_dense(0, gate, up, down)
    ctx.finalize_layer(0)
    del gate, up, down
    for l in range(1, n):
        wl.upload_moe_layer(ctx, l, wl.moe_layer(wl.MASTER_SEED, l, dims))
    ones = np.ones(dims.hidden, np.float32)
    for l in range(n):
        ctx.upload_norm(l, ones)
    resident = ctx.resident_bytes()
    out = {"layers": n, "resident_gb": round(resident / 1e9, 2)}
    for T, steps in ((1, steps_t1), (big_tokens, steps_big)):
        h0 = wl.tokens(wl.MASTER_SEED + 11, T, dims.hidden)
        dh = ctx.to_device(h0)
        for _ in range(2):  # warm-up passes (the hidden state keeps evolving; timing only)
            ctx.stack_forward(0, n - 1, dh, T)
        ctx.synchronize()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for _ in range(steps):
            ctx.stack_forward(0, n - 1, dh, T)
        ctx.record(e1)
        ctx.synchronize()
        ms = ctx.elapsed_ms(e0, e1) / steps
        out[f"t{T}"] = {"tokens": T, "steps": steps, "ms_per_step": round(ms, 4),
                        "value": round(T / (ms / 1e3), 1), "unit": "tokens/s"}
        log(f"stack T={T}: {ms:.3f} ms per step")
        if T > 1:
            # the same pass replayed from a captured HIP graph
            graph = ctx.stack_graph_create(0, n - 1, dh, T)
            ctx.stack_graph_launch(graph)
            ctx.synchronize()
            ctx.record(e0)
            for _ in range(steps):
                ctx.stack_graph_launch(graph)
            ctx.record(e1)
            ctx.synchronize()
            gms = ctx.elapsed_ms(e0, e1) / steps
            ctx.stack_graph_destroy(graph)
            out[f"t{T}"]["graph_ms_per_step"] = round(gms, 4)
            log(f"stack T={T} as a graph: {gms:.3f} ms per step")
        dh.free()
    ctx.close()
    return out


def run_decoder(steps: int, warmup: int, moe_layers: int, context: int) -> dict:
    """DeepSeek-V2-Lite's layer loop as DeepSeekRunner::forward runs it
    (src/DeepSeekRunner.cpp:251-291), without the embedding and the LM head:
    per layer h += attention(rms_norm(h, input_norm)), then h += FFN(rms_norm(h,
    post_norm)); layer 0 dense, layers 1..`moe_layers` MoE, every weight
    synthetic and resident, through lm_decoder_forward.  Prefill: `context`
    tokens from position 0 through every layer (one batched call, timed with
    events, after one untimed run into a cleared cache).  Decode: `steps`
    single-token calls after `warmup` untimed ones, continuing from that
    prefill, so the KV caches hold context .. context + warmup + steps - 1
    tokens."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    d = wl.V2_LITE_MLA
    n = 1 + moe_layers
    if context + warmup + steps > d.max_positions:
        raise ValueError(f"decoder: {context} + {warmup} + {steps} tokens exceed the {d.max_positions}-token cache")
    log(f"decoder: generating and uploading dense + {moe_layers} MoE layers with attention")
    ctx = Context(dims.moe_config(num_layers=n))
    ctx.attention_configure(wl.mla_config(d))
    gate, up, down = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
    ctx.upload_dense(0, gate, up, down)
    ctx.finalize_layer(0)
    del gate, up, down
    for l in range(1, n):
        wl.upload_moe_layer(ctx, l, wl.moe_layer(wl.MASTER_SEED, l, dims))
        log(f"decoder: MoE layer {l} resident")
    for l in range(n):
        wl.upload_mla_layer(ctx, l, wl.mla_layer(wl.MASTER_SEED + 31, l, d))
        ctx.upload_input_norm(l, (1.0 + wl.normal_f32(wl.MASTER_SEED + 32, l, 0.1, (dims.hidden,))).astype(np.float32))
        ctx.upload_norm(l, (1.0 + wl.normal_f32(wl.MASTER_SEED + 33, l, 0.1, (dims.hidden,))).astype(np.float32))
    out = {"layers": n, "resident_gb": round(ctx.resident_bytes() / 1e9, 2), "context": context}
    h0 = wl.tokens(wl.MASTER_SEED + 34, context + warmup + steps, dims.hidden)
    dh = ctx.to_device(h0)
    row = dims.hidden * 4
    for rep in range(2):  # the first pass warms up; the second is timed
        ctx.kv_cache_clear()
        dh.upload(h0)
        ctx.synchronize()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        ctx.decoder_forward(0, n - 1, dh, context, 0)
        ctx.record(e1)
        ctx.synchronize()
    pre_ms = ctx.elapsed_ms(e0, e1)
    out["prefill"] = {"tokens": context, "ms": round(pre_ms, 3), "tokens_per_s": round(context / pre_ms * 1e3, 1)}
    log(f"decoder prefill T={context}: {pre_ms:.3f} ms")
    pos = context
    for _ in range(warmup):
        ctx.decoder_forward(0, n - 1, dh.ptr + pos * row, 1, pos)
        pos += 1
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(steps):
        ctx.decoder_forward(0, n - 1, dh.ptr + pos * row, 1, pos)
        pos += 1
    ctx.record(e1)
    ctx.synchronize()
    us = ctx.elapsed_ms(e0, e1) * 1e3 / steps
    out["decode"] = {"context": [context + warmup, context + warmup + steps - 1], "us_per_token": round(us, 2),
                     "us_per_layer": round(us / n, 2), "tokens_per_s": round(1e6 / us, 1)}
    log(f"decoder decode: {us:.2f} us per token ({us / n:.2f} per layer)")
    dh.free()
    ctx.close()
    return out


def cpu_layout() -> dict:
    """The host CPU as /proc/cpuinfo describes it: model, sockets x cores x SMT."""
    model, sockets, cores, siblings = None, set(), None, None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, value = line.partition(":")
                key, value = key.strip(), value.strip()
                if key == "model name" and model is None:
                    model = value
                elif key == "physical id":
                    sockets.add(value)
                elif key == "cpu cores" and cores is None:
                    cores = int(value)
                elif key == "siblings" and siblings is None:
                    siblings = int(value)
    except OSError:
        pass
    n_sockets = max(len(sockets), 1)
    smt = siblings // cores if cores and siblings else None
    return {"model": model, "sockets": n_sockets, "cores_per_socket": cores, "threads_per_core": smt,
            "layout": f"{n_sockets} x {cores} x {smt}", "online_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


def cpu_baseline(layers, x, bias, run_seconds: float, runs: int = 5, what: str = "") -> dict | None:
    """LiteMind's CPU MoE path (its own Gemm/MoeRouter/ThreadPool compiled from
    its sources into oracle/_ref, -O3 -march=x86-64-v3) on distinct tokens of
    the workload, one token at a time as its runner does (src/DeepSeekRunner.cpp:
    472-482), with ThreadPool's hardware_concurrency() workers.  Token j of the
    sample runs on layers[j % len(layers)], as the GPU leg rotates its layers.
    One warm-up run, then `runs` timed runs of distinct tokens; the value is
    tokens / median run time."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol

    if not ol.have_ref():
        return None
    threads = int(ol.ref().ref_hardware_threads())

    def run(rows):
        t0 = time.perf_counter()
        for j in rows:
            ol.ref_moe_layer(layers[j % len(layers)], x[j:j + 1], bias, workers=0)
        return time.perf_counter() - t0

    probe = run(range(min(4, x.shape[0])))  # warm-up: pool start, page-in, rate estimate
    per_token = probe / min(4, x.shape[0])
    n = int(max(4, min(x.shape[0] // (runs + 1), run_seconds / per_token)))
    run(range(n))  # warm-up run at the timed size
    times = [run(range((r + 1) * n, (r + 2) * n)) for r in range(runs)]
    median = float(np.median(times))
    return dict(value=n / median, unit="tokens/s", cores=threads, kind="reference",
                sample=f"{what}: {runs} runs of {n} distinct tokens each (after a warm-up run), median "
                       f"{median:.2f} s per run; sequential per-token MoE block with LiteMind's "
                       f"gemm/MoeRouter/ThreadPool compiled -O3 -march=x86-64-v3, {threads} threads; "
                       f"run times {', '.join(f'{t:.2f}' for t in times)} s",
                cpu=cpu_layout())


def roofline(res: dict, mfma: bool) -> dict:
    """Dominant kernel's achieved rate: algorithmic bytes (or flops) / event-timed duration."""
    alg = algorithmic(res["T"], int(round(res["distinct"])))
    if res["T"] == 1:
        # The single-token forward is one kernel (decode_fused_kernel) per step:
        # its average duration is the event-timed span of the timed steps / steps.
        dur_us = res["gpu_ms"] * 1e3 / res["steps"]
        by = alg["layer_bytes"]
        achieved = by / (dur_us * 1e-6) / 1e9
        return {"bound": "hbm", "kernel": "decode_fused_kernel", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": MEASURED_TRAFFIC.get((res["workload"], "decode_fused_kernel")),
                "avg_us": round(dur_us, 2), "algorithmic_bytes": by}
    stages = res["stages"]
    per = {k: (v[0] / v[1] if v[1] else 0.0) for k, v in stages.items()}
    dominant = max(("gate_up", "down"), key=lambda k: per[k])
    dur_s = per[dominant] / 1e3
    alg = algorithmic(res["T"], int(round(res["distinct"])), 2 if mfma else 4)
    by, fl = alg[f"{dominant}_bytes"], alg[f"{dominant}_flops"]
    gbs, tfs = by / dur_s / 1e9, fl / dur_s / 1e12
    # The bound is the resource whose peak gives the longer floor for this
    # launch (the GEMV path's fp32 VALU work never does at its token counts).
    mfma_bound = mfma and fl / (MFMA_PEAK_TFLOPS * 1e12) > by / (HBM_PEAK_GBS * 1e9)
    out = {"bound": "mfma" if mfma_bound else "hbm", "kernel": dominant}
    if mfma_bound:
        out.update(achieved=round(tfs, 2), peak=MFMA_PEAK_TFLOPS, unit="TFLOP/s", frac=round(tfs / MFMA_PEAK_TFLOPS, 4))
    else:
        out.update(achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4))
    out.update(traffic=MEASURED_TRAFFIC.get((res["workload"], dominant)), avg_us=round(per[dominant] * 1e3, 2),
               algorithmic_bytes=by, algorithmic_flops=fl, hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
    if mfma:
        out["mfma_frac"] = round(tfs / MFMA_PEAK_TFLOPS, 4)
        clk = res.get("clock")
        if clk:
            # the same rate against the peak at the measured clock: the share
            # of the matrix cores' issue slots the kernel fills
            out["clock_mhz"] = clk["mhz"]
            out["mfma_frac_at_clock"] = round(tfs / (MFMA_PEAK_TFLOPS * clk["mhz"] / PEAK_CLOCK_MHZ), 4)
    return out


def swiglu(res: dict) -> dict:
    """The grouped SwiGLU (gate/up and down launches together) against dense MFMA peak."""
    stages = res["stages"]
    us = sum(stages[k][0] / stages[k][1] * 1e3 for k in ("gate_up", "down") if stages.get(k) and stages[k][1])
    alg = algorithmic(res["T"], int(round(res["distinct"])))
    fl = alg["gate_up_flops"] + alg["down_flops"]
    tf = fl / (us * 1e-6) / 1e12 if us else 0.0
    traffic = [MEASURED_TRAFFIC.get((res["workload"], k)) for k in ("gate_up", "down")]
    out = {"us": round(us, 2), "flops": fl, "achieved": round(tf, 2), "unit": "TFLOP/s", "peak": MFMA_PEAK_TFLOPS,
           "frac": round(tf / MFMA_PEAK_TFLOPS, 4), "traffic": None if None in traffic else sum(traffic)}
    clk = res.get("clock")
    out["clock"] = clk
    if clk:
        out["peak_at_clock"] = round(MFMA_PEAK_TFLOPS * clk["mhz"] / PEAK_CLOCK_MHZ, 1)
        out["frac_at_clock"] = round(tf / out["peak_at_clock"], 4) if tf else 0.0
    return out


def run_load(moe_layers: int) -> dict:
    """Checkpoint to HBM: writes DeepSeek-V2-Lite's dense layer 0 and `moe_layers`
    MoE layers as SafeTensors shards (one per layer, DeepSeek's tensor names) into a
    temporary directory, then times lm_checkpoint_open and lm_load_layer per layer
    (header validation, the gate/up interleave on the host, the copy to HBM and the
    fp16 shadow).  The shards were just written, so they are read from the page
    cache, not from disk.  (Parity: tests/test_gpu_checkpoint.py.)"""
    import tempfile

    from litemind_amd import Checkpoint, Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    n = 1 + moe_layers
    ones = np.ones(dims.hidden, np.float32)
    with tempfile.TemporaryDirectory(prefix="lm_ckpt_") as d:
        log(f"load: writing dense + {moe_layers} MoE layer shards")
        wl.save_safetensors(os.path.join(d, "model-00000.safetensors"),
                            wl.dense_layer_tensors(0, wl.dense_ffn(wl.MASTER_SEED, 0, dims), ones))
        for l in range(1, n):
            wl.save_safetensors(os.path.join(d, f"model-{l:05d}.safetensors"),
                                wl.moe_layer_tensors(l, wl.moe_layer(wl.MASTER_SEED, l, dims), ones))
        shard_bytes = sum(os.path.getsize(os.path.join(d, f)) for f in os.listdir(d))
        ctx = Context(dims.moe_config(num_layers=n))
        t0 = time.perf_counter()
        ck = Checkpoint(d)
        t_open = time.perf_counter() - t0
        per_layer = []
        for l in range(n):
            t1 = time.perf_counter()
            ctx.load_layer(ck, l)
            ctx.synchronize()
            per_layer.append(time.perf_counter() - t1)
            log(f"load: layer {l} {per_layer[-1] * 1e3:.1f} ms")
        total = time.perf_counter() - t0
        tensors, shards = ck.count()
        ck.close()
        resident = ctx.resident_bytes()
        ctx.close()
    return {"layers": n, "tensors": tensors, "shards": shards, "shard_bytes": shard_bytes,
            "resident_bytes": resident, "open_ms": round(t_open * 1e3, 2),
            "layer_ms": [round(t * 1e3, 1) for t in per_layer], "total_s": round(total, 3),
            "value": round(shard_bytes / total / 1e9, 3), "unit": "GB/s"}


MLA_CACHE_BYTES_PER_TOKEN = 4 * (16 * (128 + 128) + 64)  # 16,640: fp32 key_nope, value, key_rope


def mla_projection_bytes(d) -> int:
    """BF16 bytes of one attention layer's projections (q without LoRA)."""
    q = d.heads * d.qk_head * d.hidden
    kv_a = (d.kv_lora_rank + d.qk_rope) * d.hidden
    kv_b = d.heads * (d.qk_nope + d.v_head) * d.kv_lora_rank
    o = d.hidden * d.heads * d.v_head
    return 2 * (q + kv_a + kv_b + o)


def run_attention(steps: int, warmup: int) -> dict:
    """One DeepSeek-V2-Lite attention layer (multi-head latent attention, q
    without LoRA, YaRN rotary, 4096-token KV cache) resident in HBM.  Decode:
    `steps` single-token calls after `warmup` untimed ones, the cache filled
    before them by a batched prefill to `start` tokens, so the timed steps see
    contexts start .. start + steps - 1.  Prefill: 512 tokens from position 0
    (causal) into an emptied cache, each call timed with events.  A decode step
    reads the projections and the whole cache once (LiteMind's KvCache holds
    fp32 per-head keys and values)."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    d = wl.V2_LITE_MLA
    H = d.hidden
    log("attention: uploading one V2-Lite attention layer")
    ctx = Context(wl.V2_LITE.moe_config(num_layers=1))
    ctx.attention_configure(wl.mla_config(d))
    wl.upload_mla_layer(ctx, 0, wl.mla_layer(wl.MASTER_SEED, 0, d))
    cap = d.max_positions
    if steps + warmup > cap - 600:
        raise ValueError(f"attention: at most {cap - 600 - warmup} decode steps fit the {cap}-token cache")
    xs = ctx.to_device(wl.tokens(wl.MASTER_SEED + 21, cap, H))
    dout = ctx.empty((cap, H))
    row = H * 4
    proj = mla_projection_bytes(d)
    out = {"projection_bytes": proj, "cache_bytes_per_token": MLA_CACHE_BYTES_PER_TOKEN}
    for start in (512, cap - steps - 56):
        ctx.kv_cache_clear()
        pos = start - warmup
        for p0 in range(0, pos, 512):
            n = min(512, pos - p0)
            ctx.attention_forward(0, xs.ptr + p0 * row, n, p0, dout.ptr + p0 * row)
        for i in range(warmup):
            ctx.attention_forward(0, xs.ptr + pos * row, 1, pos, dout.ptr + pos * row)
            pos += 1
        ctx.synchronize()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for i in range(steps):
            ctx.attention_forward(0, xs.ptr + pos * row, 1, pos, dout.ptr + pos * row)
            pos += 1
        ctx.record(e1)
        ctx.synchronize()
        us = ctx.elapsed_ms(e0, e1) * 1e3 / steps
        by = proj + (start + (steps - 1) / 2 + 1) * MLA_CACHE_BYTES_PER_TOKEN + 2 * row
        out[f"decode_ctx{start}"] = {"context": [start, start + steps - 1], "us_per_step": round(us, 2),
                                     "tokens_per_s": round(1e6 / us, 1), "bytes_per_step": int(by),
                                     "achieved_gbs": round(by / us / 1e3, 1),
                                     "hbm_frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"attention decode from context {start}: {us:.2f} us per step")
    T = 512
    times = []
    for i in range(warmup + 10):
        ctx.kv_cache_clear()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        ctx.attention_forward(0, xs, T, 0, dout)
        ctx.record(e1)
        ctx.synchronize()
        if i >= warmup:
            times.append(ctx.elapsed_ms(e0, e1) * 1e3)
    us = float(np.median(times))
    out["prefill_t512"] = {"tokens": T, "us": round(us, 2), "tokens_per_s": round(T / us * 1e6, 1)}
    log(f"attention prefill T={T}: {us:.2f} us")
    xs.free()
    dout.free()
    ctx.close()
    return out


def run_head(steps: int, warmup: int) -> dict:
    """DeepSeek-V2-Lite's final norm and LM head ([102400, 2048] BF16, resident)
    for one token, then the greedy next token: lm_head_forward, timed with events
    on the library's stream.  (Parity: tests/test_gpu_head.py.)"""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    V, H = 102400, dims.hidden
    ctx = Context(dims.moe_config(num_layers=1))
    rng = np.random.default_rng(wl.MASTER_SEED)
    log("head: generating and uploading the [102400, 2048] head")
    ctx.upload_head(np.ones(H, np.float32), wl.normal_bf16(wl.MASTER_SEED, 7777, 0.02, (V, H)))
    dh = ctx.to_device(rng.standard_normal((1, H)).astype(np.float32))
    tok = ctx.empty((1,), np.int32)
    for _ in range(warmup):
        ctx.head_forward(dh, 1, token=tok)
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(steps):
        ctx.head_forward(dh, 1, token=tok)
    ctx.record(e1)
    ctx.synchronize()
    us = ctx.elapsed_ms(e0, e1) * 1e3 / steps
    ctx.close()
    head_bytes = V * H * 2 + H * 4 * 2 + V * 4  # head, hidden + norm weight, logits written
    tbs = head_bytes / (us * 1e-6) / 1e12
    return {"us": round(us, 2), "bytes": head_bytes, "achieved": round(tbs * 1e3, 1), "unit": "GB/s",
            "peak": HBM_PEAK_GBS, "frac": round(tbs * 1e3 / HBM_PEAK_GBS, 4)}


def run_v2_decode(steps: int, warmup: int, rotate: int, prefill: bool = True) -> dict:
    """DeepSeek-V2's full MoE layer (hidden 5120, 160 routed experts in 8
    groups of which 3 are kept, top-6, two shared experts of 1536, routed
    weights scaled by 16) at T = 1, `rotate` independently seeded layers
    resident (15.1 GB each with the fp16 shadow) and rotated per step.  Its
    shape is outside the single-token kernel's (more than 64 experts, hidden
    above 4096), so LM_PATH_AUTO runs the router (MoeRouter's group mask) and
    the gate/up projections as one speculative launch, then the GEMV down
    launch and the combine.  Per-stage times from a second pass with events
    between the stages (the speculative launch counts as the router stage)."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_FULL
    ctx = Context(dims.moe_config(num_layers=rotate))
    for l in range(rotate):
        log(f"decode_t1_v2: generating and uploading layer {l} ({dims.expert_bytes() * dims.experts / 1e9:.1f} GB BF16)")
        L = wl.moe_layer(wl.MASTER_SEED + 300 + l, 0, dims)
        wl.upload_moe_layer(ctx, l, L)
        del L
    dx = ctx.to_device(wl.tokens(wl.MASTER_SEED + 301, 1, dims.hidden))
    dy = ctx.empty((1, dims.hidden))
    didx = ctx.empty((rotate, dims.top_k), np.int32)

    def step(i):
        l = i % rotate
        ctx.moe_forward(l, dx, 1, dy, idx=didx.ptr + l * dims.top_k * 4)

    for i in range(warmup):
        step(i)
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for i in range(steps):
        step(i)
    ctx.record(e1)
    ctx.synchronize()
    us = ctx.elapsed_ms(e0, e1) * 1e3 / steps
    ctx.stage_timing(True)
    for i in range(steps):
        step(i)
    stages = {k: round(v[0] * 1e3 / v[1], 2) if v[1] else None for k, v in ctx.stage_times().items()}
    ctx.stage_timing(False)
    idx = didx.download()
    H, I, S, E = dims.hidden, dims.inter, dims.shared_inter, dims.experts
    by = 6 * 3 * I * H * 2 + 3 * S * H * 2 + E * H * 4 + H * 8
    gbs = by / (us * 1e-6) / 1e9
    out = {"us": round(us, 2), "tokens_per_s": round(1e6 / us, 1), "stage_us": stages,
           "algorithmic_bytes": by, "achieved": round(gbs, 1), "unit": "GB/s", "peak": HBM_PEAK_GBS,
           "frac": round(gbs / HBM_PEAK_GBS, 4), "experts_per_step": [sorted(map(int, r)) for r in idx]}
    if not prefill:
        ctx.close()
        return out
    # a prefill batch of 2048 tokens on layer 0 (MFMA experts): stage times
    T = 2048
    dxp = ctx.to_device(wl.tokens(wl.MASTER_SEED + 302, T, dims.hidden))
    dyp = ctx.empty((T, dims.hidden))
    for _ in range(5):
        ctx.moe_forward(0, dxp, T, dyp)
    ctx.synchronize()
    ctx.record(e0)
    for _ in range(10):
        ctx.moe_forward(0, dxp, T, dyp)
    ctx.record(e1)
    ctx.synchronize()
    us_p = ctx.elapsed_ms(e0, e1) * 1e3 / 10
    ctx.stage_timing(True)
    for _ in range(10):
        ctx.moe_forward(0, dxp, T, dyp)
    stages_p = {k: round(v[0] * 1e3 / v[1], 2) if v[1] else None for k, v in ctx.stage_times().items()}
    ctx.stage_timing(False)
    ctx.close()
    out["t2048"] = {"us": round(us_p, 2), "tokens_per_s": round(T / (us_p * 1e-6), 1), "stage_us": stages_p}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="decode_t1")
    ap.add_argument("--second", default="prefill_t2048_skewed", help="second workload ('' to skip)")
    ap.add_argument("--rotate", type=int, default=8, help="layers rotated through at T=1")
    ap.add_argument("--path", type=int, default=0, help="0 auto, 1 GEMV, 2 MFMA")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-v2", action="store_true",
                    help="skip the default run's DeepSeek-V2 T=1 leg (160 experts: the speculative launch)")
    args = ap.parse_args()
    if args.workload == "stack":
        if args.gpus != 1:
            print("bench.py measures one GPU.", file=sys.stderr)
            return 2
        st = run_stack(args.steps if args.steps != 200 else 20, 5, 4096, 26)
        line = {"metric": "MoE FFN stack tokens/sec (dense layer 0 + 26 MoE layers, RMSNorm-chained)",
                "value": st["t1"]["value"], "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True,
                "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) RMS-normalised tokens)",
                "config": {"workload": "stack", "layers": st["layers"], "resident_gb": st["resident_gb"]},
                "t1": st["t1"], "t4096": st["t4096"]}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "attention":
        if args.gpus != 1:
            print("bench.py measures one GPU.", file=sys.stderr)
            return 2
        at = run_attention(args.steps, args.warmup)
        main = at[max((k for k in at if k.startswith("decode_ctx")), key=lambda k: int(k[len("decode_ctx"):]))]
        line = {"metric": "MLA attention decode tokens/sec (one V2-Lite layer, KV cache near 4K tokens)",
                "value": main["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": round(main["us_per_step"] / 1e3, 5), "higher_is_better": True,
                "dtype": "fp32", "data": "synthetic (seeded N(0,0.02) BF16 projections, N(0,1) RMS-normalised tokens)",
                "config": {"workload": "attention", "hidden": 2048, "heads": 16, "kv_lora_rank": 512,
                           "qk_nope": 128, "qk_rope": 64, "v_head": 128, "cache_tokens": 4096},
                "roofline": {"bound": "hbm", "achieved": main["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": main["hbm_frac"], "traffic": None, "avg_us": main["us_per_step"],
                             "algorithmic_bytes": main["bytes_per_step"]},
                "attention": at}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "decoder":
        if args.gpus != 1:
            print("bench.py measures one GPU.", file=sys.stderr)
            return 2
        dc = run_decoder(args.steps if args.steps != 200 else 100, args.warmup, 26, 512)
        line = {"metric": "DeepSeek-V2-Lite decoder layers, decode tokens/sec (27 layers of attention + FFN, "
                          "KV cache near 512 tokens)",
                "value": dc["decode"]["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
                "steps": args.steps if args.steps != 200 else 100, "warmup": args.warmup,
                "ms_per_step": round(dc["decode"]["us_per_token"] / 1e3, 5), "higher_is_better": True,
                "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) tokens)",
                "config": {"workload": "decoder", "layers": dc["layers"], "resident_gb": dc["resident_gb"],
                           "prefill_tokens": dc["context"]},
                "decoder": dc}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "head":
        if args.gpus != 1:
            print("bench.py measures one GPU.", file=sys.stderr)
            return 2
        hd = run_head(args.steps, args.warmup)
        line = {"metric": "LM head + greedy next token, tokens/sec (V=102400, H=2048)",
                "value": round(1e6 / hd["us"], 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": round(hd["us"] / 1e3, 5), "higher_is_better": True,
                "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) head)",
                "config": {"workload": "head", "vocab": 102400, "hidden": 2048},
                "roofline": {"bound": "hbm", "achieved": hd["achieved"], "peak": hd["peak"], "unit": "GB/s",
                             "frac": hd["frac"], "traffic": None, "avg_us": hd["us"], "algorithmic_bytes": hd["bytes"]}}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "decode_t1_v2":
        if args.gpus != 1:
            print("bench.py measures one GPU.", file=sys.stderr)
            return 2
        v2 = run_v2_decode(args.steps, args.warmup, min(args.rotate, 4))
        line = {"metric": "DeepSeek-V2 MoE-layer tokens/sec at T=1 (160 experts in 8 groups, hidden 5120)",
                "value": v2["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": round(v2["us"] / 1e3, 5), "higher_is_better": True,
                "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) RMS-normalised tokens)",
                "config": {"workload": "decode_t1_v2", "tokens": 1, "hidden": 5120, "experts": 160, "top_k": 6,
                           "n_group": 8, "topk_group": 3, "moe_intermediate": 1536, "shared_intermediate": 3072,
                           "layers_rotated": min(args.rotate, 4)},
                "roofline": {"bound": "hbm", "achieved": v2["achieved"], "peak": v2["peak"], "unit": "GB/s",
                             "frac": v2["frac"], "traffic": None, "avg_us": v2["us"],
                             "algorithmic_bytes": v2["algorithmic_bytes"]},
                "stage_us": v2["stage_us"], "experts_per_step": v2["experts_per_step"], "t2048": v2["t2048"]}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "load":
        if args.gpus != 1:
            print("bench.py measures one GPU.", file=sys.stderr)
            return 2
        ld = run_load(3)
        line = {"metric": "SafeTensors checkpoint to HBM (shard bytes per second, page-cache-warm)",
                "value": ld["value"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "dtype": "bf16",
                "data": "synthetic (seeded N(0,0.02) weights written as SafeTensors shards)",
                "config": {"workload": "load", "layers": ld["layers"], "shards": ld["shards"],
                           "tensors": ld["tensors"]}, "load": ld}
        print(json.dumps(line), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path (asked for {args.gpus}).",
              file=sys.stderr)
        return 2

    import litemind_amd as lm
    from litemind_amd import workload as wl

    main_w = wl.WORKLOADS[args.workload]
    rotate = args.rotate if main_w.tokens <= 64 else 1
    res = run_gpu(args.workload, args.steps, args.warmup, rotate, args.path)
    T = res["T"]
    ms = res["wall_s"] * 1e3 / res["steps"]
    mfma_main = T > lm.MFMA_CROSSOVER if args.path == 0 else args.path == 2
    line = {
        "metric": METRIC, "value": round(T / (ms / 1e3), 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) RMS-normalised tokens)",
        "config": {"workload": args.workload, "tokens": T, "hidden": 2048, "experts": 64, "top_k": 6,
                   "moe_intermediate": 1408, "shared_intermediate": 2816, "layers_rotated": rotate,
                   "expert_path": "mfma-fp16" if mfma_main else "gemv-fp32",
                   "distinct_experts_per_step": res["distinct"]},
        "roofline": roofline(res, mfma_main),
        "layer_gpu_us": round(res["gpu_ms"] * 1e3 / res["steps"], 2),
        "clock": res["clock"],
        "clock_amdsmi": res.get("clock_amdsmi"),
    }
    if res["stages"]:
        line["stage_us"] = {k: round(v[0] * 1e3 / v[1], 2) if v[1] else None for k, v in res["stages"].items()}
    alg = algorithmic(T, int(round(res["distinct"])))
    line["layer_hbm_frac"] = round(alg["layer_bytes"] / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)

    if not args.no_cpu:
        log("cpu baseline (LiteMind's own kernels)")
        if T == 1:
            # distinct tokens drawn like the workload's, layers rotated as the GPU leg rotates them
            x_cpu = wl.tokens(wl.MASTER_SEED + 8, 8192, 2048)
            what = (f"decode: tokens from a seeded N(0,1) RMS-normalised stream, layers rotated over the "
                    f"{len(res['layers'])} benchmark layers")
        else:
            x_cpu = res["x"]
            what = f"{args.workload}: distinct rows of the workload's {T} tokens"
        cb = cpu_baseline(res["layers"], x_cpu, res["bias"], args.cpu_seconds / 5, what=what)
        if cb is None:
            cb = {"value": None, "unit": "tokens/s", "cores": os.cpu_count(), "kind": "reference",
                  "sample": "oracle/_ref/libref.so not built"}
        line["cpu_baseline"] = cb

    if args.second:
        w2 = wl.WORKLOADS[args.second]
        # 30 warm-up steps: after the single-token phase the heavy launches
        # need ~25 steps to settle (measured: 586 us per step over the first 20
        # steps after 5 warm-up steps, 515-518 us from then on, and the
        # kernels' own durations fall over the same launches).
        res2 = run_gpu(args.second, max(10, args.steps // 10), max(30, args.warmup // 4), 1, args.path)
        ms2 = res2["wall_s"] * 1e3 / res2["steps"]
        mfma2 = w2.tokens > lm.MFMA_CROSSOVER if args.path == 0 else args.path == 2
        line["t2048" if w2.tokens == 2048 else args.second] = {
            "workload": args.second, "tokens": w2.tokens, "value": round(w2.tokens / (ms2 / 1e3), 1),
            "unit": "tokens/s", "ms_per_step": round(ms2, 4), "steps": res2["steps"],
            "expert_path": "mfma-fp16" if mfma2 else "gemv-fp32",
            "roofline": roofline(res2, mfma2),
            "stage_us": {k: round(v[0] * 1e3 / v[1], 2) if v[1] else None for k, v in res2["stages"].items()},
            "clock": res2["clock"],
            "clock_amdsmi": res2.get("clock_amdsmi"),
        }
        if mfma2:
            line["t2048" if w2.tokens == 2048 else args.second]["grouped_swiglu"] = swiglu(res2)
        if not args.no_cpu:
            log(f"cpu baseline on a sample of {args.second}")
            cb2 = cpu_baseline(res2["layers"], res2["x"], res2["bias"], args.cpu_seconds / 12,
                               what=f"{args.second}: distinct rows of the workload's {w2.tokens} tokens")
            if cb2 is not None:
                line["t2048" if w2.tokens == 2048 else args.second]["cpu_baseline"] = cb2
    if not args.no_v2 and args.workload == "decode_t1":
        # DeepSeek-V2's MoE layer (160 experts in 8 groups, hidden 5120) at T = 1:
        # more experts than the single-token kernel's lanes, so the router and
        # gate/up run as one speculative launch, then down and the combine
        log("decode_t1_v2 leg: DeepSeek-V2 layers at T=1 (4 rotated)")
        v2 = run_v2_decode(args.steps, args.warmup, 4, prefill=False)
        line["deepseek_v2_t1"] = {
            "workload": "decode_t1_v2", "tokens": 1, "hidden": 5120, "experts": 160, "top_k": 6, "n_group": 8,
            "topk_group": 3, "layers_rotated": 4, "us": v2["us"], "value": v2["tokens_per_s"],
            "unit": "tokens/s", "steps": args.steps,
            "roofline": {"bound": "hbm", "achieved": v2["achieved"], "peak": v2["peak"], "unit": "GB/s",
                         "frac": v2["frac"], "algorithmic_bytes": v2["algorithmic_bytes"]},
            "stage_us": v2["stage_us"]}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
