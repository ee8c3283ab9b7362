"""Benchmark of the full-attention hot path on one MI355X.

Default run: both halves of the headline metric in one JSON line.

- Decode: batch-1 GQA decode, 24 q heads / 4 kv
  heads, head_dim 256, 32768 keys of q8_0 K/V (N(0,1) plus one x8 outlier dim
  per head). One step is one token through the reference model's 16
  full-attention layers: per layer, one rd4_attn_decode_append launch
  (append-and-quantize of the token's K/V rows at position 32767 + gated
  split-KV attention over keys 0..32767) on that layer's own cache. The 16
  caches (1.14 GB) are larger than the 256 MB MALL, so every layer reads its
  cache from HBM, as in a real decode step. The 16 launches are replayed as one
  HIP graph (eager launches when --eager).
- Prefill, under "prefill": 4096 f16 queries over 4096 + 4096
  f16 keys, causal, gated, with the chunk's K/V rows appended as q8_0 in the
  same rd4_prefill_append launch.

value = algorithmic bytes of a step / step time (GB/s). "hbm_read_ceiling" is
the same run's measurement of a launch that only streams the same bytes
(rd4_read_probe, 16 HBM-true launches per step): the practical ceiling beside
the 8 TB/s peak. Each roofline object
covers that half's dominant kernel, timed with HIP events on the stream the
library launches on. cpu_baseline = the scalar CPU oracle (f64, one thread) on
a bounded sample of the same workload. "prefill" also carries
"reference_chunks": the same chunk as 8 calls of 512 queries, the shape the
reference engine issues. "extra" holds the other decode configs (f16 32K, q4_0
131K, the q5_0/q4_1 131K pair, the 4-token MTP verify step), each with its own
roofline (`--no-extra` skips them). `--workload X` measures one workload alone
(for profiling).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
NH, NKV, HD = 24, 4, 256
SEED = 20260


def pkg():
    import importlib.util
    name = "rdna4_infer_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "rdna4-infer_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def make_cache(torch, rd4, t, n, seed, outlier):
    """n rows x 4 kv heads of N(0,1) values (optionally one x8 dim per head),
    quantized on the GPU by the library's own store kernel."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    rb = rd4.kv_row_bytes(t, HD)
    cache = torch.empty(n * NKV * rb, dtype=torch.uint8, device="cuda")
    step = 4096
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        x = torch.randn((r1 - r0, NKV, HD), generator=g, device="cuda", dtype=torch.float32)
        if outlier:
            x[:, :, 7] *= 8
        rd4.kv_store_rows(t, x.reshape(-1), cache[r0 * NKV * rb:r1 * NKV * rb])
    return cache


def measured_traffic(workload):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE passes (profiles/traffic.json, copy-calibrated), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[workload]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def event_loop_ms(torch, fn, steps):
    """Mean ms per call of fn() over `steps` back-to-back calls, from two HIP
    events recorded on the current stream (the stream the library launches on)
    around the whole loop: per-launch gaps overlap the previous kernel, as in a
    decode loop, so this is the kernel's sustained duration."""
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / steps


def decode_workload(torch, rd4, kt, ctx, outlier, gated=True, vt=None, layers=16):
    """One decode token through `layers` attention layers, each with its own K/V
    cache of `ctx` rows and its own q / gate / out / new rows.

    Returns (step_fn, dominant_fn, step bytes, dominant bytes, cpu_fn, info);
    the dominant kernel is the attention launch itself (one per layer), so
    both are the same function here."""
    vt = kt if vt is None else vt
    pos = ctx - 1
    krb, vrb = rd4.kv_row_bytes(kt, HD), rd4.kv_row_bytes(vt, HD)
    g = torch.Generator(device="cuda").manual_seed(SEED + 2)
    L = []
    for l in range(layers):
        kc = make_cache(torch, rd4, kt, ctx, SEED + 10 * l, outlier)
        vc = make_cache(torch, rd4, vt, ctx, SEED + 10 * l + 1, outlier)
        q = torch.randn(NH * HD, generator=g, device="cuda")
        gate = torch.randn(NH * HD, generator=g, device="cuda")
        krow = torch.randn(NKV * HD, generator=g, device="cuda")
        vrow = torch.randn(NKV * HD, generator=g, device="cuda")
        out = torch.empty(NH * HD, device="cuda")
        L.append((q, gate, krow, vrow, kc, vc, out))
    scale = 1.0 / np.sqrt(HD)

    def step():
        # per layer, one launch: quantize-append the token's K/V rows at `pos`,
        # then gated attention over keys 0..pos of that layer's cache
        for (q, gate, krow, vrow, kc, vc, out) in L:
            rd4.attn_decode_append(q, krow, vrow, kc, vc, out, pos, NH, NKV, HD, scale, kt, vt,
                                   gate=gate if gated else None)

    kv_bytes = ctx * NKV * (krb + vrb)
    small = NH * HD * 4 * (4 if gated else 2)  # q, out (+ gate read and write)
    append = 2 * NKV * HD * 4 + NKV * (krb + vrb)
    layer_bytes = kv_bytes + small + append  # the append is inside the attention launch
    step_bytes = layers * layer_bytes

    def cpu(budget_s=12.0, threads=1):
        """f64 oracle on layer 0's cache, repeated for ~budget_s; returns GB/s
        (bytes of one layer over the time of one layer). threads > 1 runs its
        OpenMP form (parallel over heads)."""
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        q, gate, krow, vrow, kc, vc, out = L[0]
        kh, vh = kc.cpu().numpy(), vc.cpu().numpy()
        qh = q.cpu().numpy()
        reps, t0 = 0, time.perf_counter()
        while True:
            orc.attn_decode(qh, kh, vh, pos, NH, NKV, HD, scale, kt, vt, threads=threads)
            reps += 1
            if time.perf_counter() - t0 > budget_s:
                break
        dt = (time.perf_counter() - t0) / reps
        return layer_bytes / dt / 1e9, "one layer's decode over %d keys x %d reps" % (ctx, reps)

    kv_name = rd4.TYPE_NAMES[kt] if kt == vt else rd4.TYPE_NAMES[kt] + "/" + rd4.TYPE_NAMES[vt]
    info = {"workload": "decode", "kv_type": kv_name, "ctx": ctx, "n_head": NH,
            "n_head_kv": NKV, "head_dim": HD, "gate": gated, "append": True, "seed": SEED,
            "layers_per_step": layers, "kv_bytes_per_step": kv_bytes * layers}
    return step, step, step_bytes, step_bytes, cpu, info


def tokens_workload(torch, rd4, kt=2, ctx=32768, n_tok=4, layers=16):
    """MTP verify step: per layer, n_tok consecutive tokens ending at key ctx-1
    attend (gated) in one rd4_attn_decode_tokens launch, each layer over its own
    cache; bytes = the K/V rows the tokens span, read once."""
    krb = rd4.kv_row_bytes(kt, HD)
    g = torch.Generator(device="cuda").manual_seed(SEED + 4)
    L = []
    for l in range(layers):
        kc = make_cache(torch, rd4, kt, ctx, SEED + 10 * l, True)
        vc = make_cache(torch, rd4, kt, ctx, SEED + 10 * l + 1, True)
        q = torch.randn(n_tok * NH * HD, generator=g, device="cuda")
        gate = torch.randn(n_tok * NH * HD, generator=g, device="cuda")
        L.append((q, gate, kc, vc, torch.empty_like(q)))

    def step():
        for (q, gate, kc, vc, out) in L:
            rd4.attn_decode_tokens(q, kc, vc, out, ctx - n_tok, n_tok, NH, NKV, HD, 1.0 / 16, kt, kt,
                                   gate=gate)

    kv_bytes = layers * (ctx * NKV * 2 * krb + n_tok * NH * HD * 4 * 4)
    info = {"workload": "decode_tokens", "kv_type": rd4.TYPE_NAMES[kt], "ctx": ctx, "n_tok": n_tok,
            "n_head": NH, "n_head_kv": NKV, "head_dim": HD, "gate": True, "seed": SEED,
            "layers_per_step": layers}
    return step, step, kv_bytes, kv_bytes, None, info


def prefill_workload(torch, rd4, n_prefix=4096, n_q=4096):
    """4096 f16 queries at positions 4096..8191 over an f16 cache of
    8192 rows (prefix + the chunk), causal, gated; the chunk's K/V rows are also
    appended to a q8_0 cache in the same launch (rd4_prefill_append)."""
    ktot = n_prefix + n_q
    kc = make_cache(torch, rd4, 1, ktot, SEED, False)
    vc = make_cache(torch, rd4, 1, ktot, SEED + 1, False)
    g = torch.Generator(device="cuda").manual_seed(SEED + 3)
    q = torch.randn((n_q, NH, HD), generator=g, device="cuda").half()
    gate = torch.randn((n_q, NH, HD), generator=g, device="cuda")
    knew = torch.randn(n_q * NKV * HD, generator=g, device="cuda")
    vnew = torch.randn(n_q * NKV * HD, generator=g, device="cuda")
    rb8 = rd4.kv_row_bytes(2, HD)
    kq8 = torch.empty(ktot * NKV * rb8, dtype=torch.uint8, device="cuda")
    vq8 = torch.empty_like(kq8)
    out = torch.empty((n_q, NH, HD), device="cuda")
    pairs = n_q * (n_prefix + 1) + n_q * (n_q - 1) // 2
    flops = NH * pairs * 4 * HD

    kq8_chunk, vq8_chunk = kq8[n_prefix * NKV * rb8:], vq8[n_prefix * NKV * rb8:]

    def step():
        # one launch: gated causal prefill + the chunk's K/V rows appended as q8_0
        rd4.prefill_append(q, kc, vc, out, n_prefix, NH, NKV, HD, 1.0 / 16, 1, 1, knew, vnew,
                           kq8_chunk, vq8_chunk, 2, gate=gate)
    attn = step

    # The reference engine's shape of the same work: prefill_plan caps a chunk at
    # 512 tokens (graph.cuh:1890-1939) and fa2_prefill_usable admits n_q == 512
    # (attn_fa2.cuh:192-207), so a 4096-token prompt arrives as 8 calls of 512
    # queries at pos0 = 4096 + 512 i. Same FLOPs, same outputs (bit for bit).
    kn3, vn3 = knew.view(n_q, NKV * HD), vnew.view(n_q, NKV * HD)

    def step_chunks(c=512):
        for r0 in range(0, n_q, c):
            rd4.prefill_append(q[r0:r0 + c], kc, vc, out[r0:r0 + c], n_prefix + r0, NH, NKV, HD, 1.0 / 16,
                               1, 1, kn3[r0:r0 + c], vn3[r0:r0 + c], kq8_chunk[r0 * NKV * rb8:],
                               vq8_chunk[r0 * NKV * rb8:], 2, gate=gate[r0:r0 + c])
    step.chunks = step_chunks

    def cpu(budget_s=12.0):
        """Oracle on a deterministic subset of query rows, scaled by causal pairs."""
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        kh, vh = kc.cpu().numpy(), vc.cpu().numpy()
        qh = q.float().cpu().numpy()
        rows = [0, n_q // 3, 2 * n_q // 3, n_q - 1]
        t0 = time.perf_counter()
        done_pairs = 0
        i = 0
        while time.perf_counter() - t0 < budget_s:
            r = rows[i % len(rows)]
            orc.attn_batch(qh[r:r + 1], kh, vh, [n_prefix + r], NH, NKV, HD, 1 / 16, 1, 1)
            done_pairs += n_prefix + r + 1
            i += 1
        dt = time.perf_counter() - t0
        return NH * done_pairs * 4 * HD / dt / 1e12, "%d query rows of the chunk, scaled by causal pairs" % i

    info = {"workload": "prefill", "kv_type": "f16", "q_type": "f16", "n_prefix": n_prefix,
            "n_q": n_q, "n_head": NH, "n_head_kv": NKV, "head_dim": HD, "causal": True,
            "gate": True, "append": "q8_0", "seed": SEED}
    return step, attn, flops, flops, cpu, info


def as_graph(torch, fn):
    """fn's launches captured once into a HIP graph (torch.cuda.CUDAGraph);
    returns its replay function, or None when capture is not possible."""
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        torch.cuda.synchronize()
        return g.replay
    except Exception as e:  # capture failed: measure eager launches instead
        print("graph capture failed (%s); timing eager launches" % e, file=sys.stderr)
        torch.cuda.synchronize()
        return None


def measure(torch, step, dominant, steps, warmup):
    """(ms per step, ms per dominant-kernel launch): the timed region is bracketed
    by synchronize() on both sides; the dominant kernel's own loop follows when
    the step holds other launches too."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_ms = event_loop_ms(torch, step, steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    dom_ms = ev_ms if dominant is step else event_loop_ms(torch, dominant, steps)
    return max(wall_ms, ev_ms), dom_ms


def decode_result(rd4, args, torch, name, graph=True):
    """Measure one decode-style workload; returns (result fields, cpu_fn)."""
    step, dom, step_units, dom_units, cpu, info = build_workload(torch, rd4, name, args)
    runner = as_graph(torch, step) if graph else None
    info["launch"] = "hip graph of the step's %d launches" % info["layers_per_step"] if runner else "eager"
    run = runner or step
    wall_ms, dom_ms = measure(torch, run, run, args.steps, args.warmup)
    nl = info["layers_per_step"]
    value = step_units / (wall_ms * 1e-3) / 1e9
    achieved = dom_units / (dom_ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(name),
            "kernel_us": round(dom_ms * 1e3 / nl, 3),
            "note": "per launch: one layer's attention (kernel_us), bytes of one layer / that time"}
    info["us_per_token_layer"] = round(wall_ms * 1e3 / nl, 3)
    return {"value": value, "wall_ms": wall_ms, "roofline": roof, "config": info}, cpu, step


def prefill_result(rd4, args, torch, one=True, chunks=True):
    """cfg 5 as one call and as the reference engine's 8 calls of 512 queries
    (one=False or chunks=False skips a half: profiling runs)."""
    step, dom, step_units, dom_units, cpu, info = build_workload(torch, rd4, "prefill", args)
    steps = max(1, min(args.steps, 50))
    if not one:
        step = dom = step.chunks
    wall_ms, dom_ms = measure(torch, step, dom, steps, min(args.warmup, 5))
    value = step_units / (wall_ms * 1e-3) / 1e12
    achieved = dom_units / (dom_ms * 1e-3) / 1e12
    roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": F16_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / F16_MFMA_PEAK_TFLOPS, 4),
            "traffic": measured_traffic("prefill"), "kernel_ms": round(dom_ms, 4)}
    # the same chunk as the reference engine issues it: 8 calls of 512 queries
    if not chunks:
        return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(wall_ms, 5),
                "roofline": roof, "workload": "prefill" if one else "prefill_chunks"}, cpu
    ch_ms, _ = measure(torch, step.chunks, step.chunks, steps, min(args.warmup, 5))
    ch = step_units / (ch_ms * 1e-3) / 1e12
    chunked = {"calls": 8, "n_q_per_call": 512, "value": round(ch, 2), "unit": "TFLOP/s",
               "ms_per_step": round(ch_ms, 5), "frac": round(ch / F16_MFMA_PEAK_TFLOPS, 4),
               "note": "configs[4] as graph.cuh:1890-1939 sends it: 8 rd4_prefill_append calls of 512 "
                       "queries at pos0 = 4096 + 512 i (same FLOPs and outputs as one call)"}
    return {"metric": "prefill attn TFLOP/s @4K causal", "value": round(value, 2), "unit": "TFLOP/s",
            "ms_per_step": round(wall_ms, 5), "steps": steps,
            "dtype": "f16 Q/K/V, f16 MFMA QK^T and PV, f32 accumulate and softmax",
            "config": info, "roofline": roof, "reference_chunks": chunked}, cpu


def read_ceiling(rd4, args, torch, steps=None):
    """Practical HBM read rate for the decode step's traffic: one streaming-read
    launch (rd4_read_probe: loads only) per layer over a buffer of a q8_0 32K
    layer's K+V bytes, `args.layers` distinct buffers (larger than the MALL),
    replayed as a HIP graph exactly like the decode step."""
    nbytes = 32768 * NKV * 272 * 2
    bufs = [torch.full((nbytes,), l, dtype=torch.uint8, device="cuda") for l in range(args.layers)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")

    def step():
        for b in bufs:
            rd4.read_probe(b, sink)
    run = as_graph(torch, step) or step
    wall_ms, _ = measure(torch, run, run, steps or args.steps, args.warmup)
    gbs = nbytes * args.layers / (wall_ms * 1e-3) / 1e9
    del bufs
    torch.cuda.empty_cache()
    # the same graph of launches over 4 KiB buffers: what a launch costs in a
    # replayed graph when it reads (almost) nothing
    tiny = [torch.full((4096,), l, dtype=torch.uint8, device="cuda") for l in range(args.layers)]

    def step0():
        for b in tiny:
            rd4.read_probe(b, sink)
    run0 = as_graph(torch, step0) or step0
    floor_ms, _ = measure(torch, run0, run0, steps or args.steps, args.warmup)
    out = {"bytes_per_launch": nbytes, "launches_per_step": args.layers,
           "us_per_launch": round(wall_ms * 1e3 / args.layers, 3), "GB/s": round(gbs, 1),
           "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "launch_floor_us": round(floor_ms * 1e3 / args.layers, 3)}
    # the probe's kernel duration from the committed rocprofv3 trace
    # (profiles/read_probe_71mb.md): the ceiling without the launch cost
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            ns = json.load(f)["read"]["avg_ns_per_step"]
        out["kernel_us_rocprof"] = round(ns / 1e3, 3)
        out["kernel_frac_of_hbm_peak"] = round(nbytes / ns / HBM_PEAK_GBS, 4)
    except (OSError, KeyError, ValueError):
        pass
    return out


def build_workload(torch, rd4, name, args):
    layers = args.layers
    if name == "decode_q8_0":
        return decode_workload(torch, rd4, 2, 32768, True, layers=layers)
    if name == "decode_f16":
        return decode_workload(torch, rd4, 1, 32768, False, layers=layers)
    if name == "decode_q4_0":
        return decode_workload(torch, rd4, 3, 131001, False, layers=max(1, layers // 4))
    if name == "decode_q5_0_q4_1":  # the reference's 131K default pair
        return decode_workload(torch, rd4, 4, 131001, False, vt=5, layers=max(1, layers // 4))
    if name == "decode_tokens":  # MTP verify: 4 tokens at 32K, q8_0
        return tokens_workload(torch, rd4, layers=layers)
    return prefill_workload(torch, rd4)


DTYPES = {
    2: "q8_0 K/V: int8 MFMA QK^T (int8 hi/lo query parts), f16 MFMA PV (f16 p*d), f32 accumulate",
    1: "f16 K/V: f16 MFMA QK^T (f16 hi/lo query parts) and PV, f32 accumulate",
    3: "q4_0 K/V: f16 MFMA on exact f16 integers, per-block f32 scales, f32 accumulate",
    4: "q5_0 K / q4_1 V: f16 MFMA on exact f16 integers, per-block f32 scales, f32 accumulate",
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="headline",
                    choices=["headline", "decode_q8_0", "decode_f16", "decode_q4_0", "decode_q5_0_q4_1",
                             "decode_tokens", "prefill", "prefill_one", "prefill_chunks", "copy", "read"])
    ap.add_argument("--layers", type=int, default=16,
                    help="attention layers (each with its own cache) per decode step")
    ap.add_argument("--eager", action="store_true", help="launch the decode step eagerly, no graph")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other decode configs (measured by default under \"extra\")")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the decode would shard "
              "by key ranges with an LSE all-gather)", file=sys.stderr)
        sys.exit(2)
    import torch
    rd4 = pkg()
    rd4.lib()
    if rd4.lib().rd4_init() != 0:
        raise SystemExit("rd4_init failed: " + rd4.lib().rd4_last_error().decode())

    if args.workload == "read":
        print(json.dumps(dict(read_ceiling(rd4, args, torch), workload="read")))
        return

    if args.workload == "copy":
        # Plain device copy of a known size: the calibration run for the
        # FETCH_SIZE / WRITE_SIZE counters (bytes read = bytes written = 256 MiB).
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        ms = event_loop_ms(torch, lambda: dst.copy_(src), args.steps)
        print(json.dumps({"workload": "copy", "bytes_read": src.numel() * 4,
                          "bytes_written": src.numel() * 4, "ms_per_copy": round(ms, 4)}))
        return

    def cpu_fields(cpu, unit, omp):
        v, sample = cpu()
        out = {"cpu_baseline": {"value": round(v, 4), "unit": unit, "cores": 1, "kind": "port",
                                "sample": sample + " (oracle/oracle.c, f64 accumulate)",
                                "host_nproc": os.cpu_count()}}
        if omp:
            # the optional multi-core form: OpenMP over heads, on the box's CPU share
            thr = max(1, min(16, os.cpu_count() or 1, NH))
            v2, sample2 = cpu(budget_s=5.0, threads=thr)
            out["cpu_baseline_omp"] = {"value": round(v2, 4), "unit": unit, "cores": thr,
                                       "kind": "port", "sample": sample2}
        return out

    if args.workload in ("prefill_one", "prefill_chunks"):  # one half alone (profiling)
        r, _ = prefill_result(rd4, args, torch, one=args.workload == "prefill_one", chunks=False)
        print(json.dumps(r))
        return
    if args.workload == "prefill":
        r, cpu = prefill_result(rd4, args, torch)
        res = dict(r, n_gpus=1, warmup=args.warmup, higher_is_better=True, scaling="weak",
                   vs_baseline=None, data="synthetic (seeded N(0,1), random K/V/Q/gate)")
        if not args.no_cpu:
            res.update(cpu_fields(cpu, "TFLOP/s", False))
        print(json.dumps(res))
        return

    name = "decode_q8_0" if args.workload == "headline" else args.workload
    r, cpu, _ = decode_result(rd4, args, torch, name, graph=not args.eager)
    info = r["config"]
    metric = "attn decode KV GB/s @32K ctx (q8_0 KV)"
    if name != "decode_q8_0":
        metric = "attn decode KV GB/s (%s, %d keys)" % (info["kv_type"], info["ctx"])
    kt = {"decode_q8_0": 2, "decode_f16": 1, "decode_q4_0": 3, "decode_q5_0_q4_1": 4}.get(name, 2)
    res = {"metric": metric, "value": round(r["value"], 3), "unit": "GB/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["wall_ms"], 5),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": DTYPES[kt],
           "data": "synthetic (seeded N(0,1), random K/V/Q/gate)", "config": info,
           "roofline": r["roofline"]}
    if not args.no_cpu and cpu is not None:
        res.update(cpu_fields(cpu, "GB/s", True))
    if name == "decode_q8_0":
        # what a launch that only streams the same bytes reaches on this GPU, in
        # the same run: the practical ceiling next to the 8 TB/s peak
        del cpu
        torch.cuda.empty_cache()
        ceil = read_ceiling(rd4, args, torch)
        ceil["decode_frac_of_ceiling"] = round(r["roofline"]["achieved"] / ceil["GB/s"], 4)
        res["hbm_read_ceiling"] = ceil
        cpu = None
    if args.workload == "headline":
        # the metric's second half: configs[4] prefill, measured in the same run
        torch.cuda.empty_cache()
        p, pcpu = prefill_result(rd4, args, torch)
        if not args.no_cpu:
            p.update(cpu_fields(pcpu, "TFLOP/s", False))
        res["prefill"] = p
    if args.workload == "headline" and not args.no_extra:
        # every other decode config of BASELINE.json (and the reference's 131K
        # default pair, and the MTP verify step), each with its own roofline
        res["extra"] = {}
        for w in ("decode_f16", "decode_q4_0", "decode_q5_0_q4_1", "decode_tokens"):
            torch.cuda.empty_cache()
            e, _, _ = decode_result(rd4, argparse.Namespace(**dict(vars(args), steps=20, warmup=3)), torch, w)
            c = e["config"]
            res["extra"][w] = {"value": round(e["value"], 1), "unit": "GB/s",
                               "us_per_token_layer": c["us_per_token_layer"],
                               "layers_per_step": c["layers_per_step"], "kv_type": c["kv_type"],
                               "ctx": c["ctx"], "roofline": e["roofline"]}
    print(json.dumps(res))


if __name__ == "__main__":
    main()
