#!/usr/bin/env python3
"""Benchmark of the paged attention path on one MI355X.

One step = one attention layer pass over one scheduler step's batch, with the step metadata
already uploaded and every input resident in HBM: the fused kernel that applies Qwen3's per-head
q/k RMSNorm, RoPE and the K/V store, then the attention kernels (split-KV decode + merge, or
MFMA prefill).

Headline (``value``): decode attention at the Qwen3-0.6B shape with 256 sequences of
log-uniform context in [128, 32768] (fragmented block tables, ~15 GB of K/V resident), in GB/s
of algorithmic bytes (each KV head's K and V rows read once, plus q/out/tables).  Reported
beside it: varlen causal prefill at the Qwen3-0.6B shape (512/1024/1536/2048, second half of
the last sequence served from 4 cached pages) in TFLOP/s of unmasked (q,k) pairs
(4 * head_dim * q_heads per pair).  Both carry a roofline object for their dominant kernel,
timed with HIP events on the library's stream during the timed region.

The CPU baseline is the oracle (a C restatement of the reference's Attention.attendJobs with its
head-major parallel split), timed on the host on a bounded sample of the same decode workload.
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "nano-vllm-java_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode-attn HBM GB/s (% of peak) + prefill-attn TFLOP/s, Qwen3-0.6B shape"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps before the timed ones; the part idles at a low clock "
                         "between phases and takes ~100 back-to-back steps of the prefill "
                         "(~30 ms) to reach its steady clock (--ramp shows it)")
    ap.add_argument("--sustain", type=float, default=0.0, metavar="S",
                    help="after the timed steps, run the step back to back for S seconds and "
                         "sample the board's socket power and gfx clock every ~10 ms (amdsmi, "
                         "when importable); the line gains their medians and ms/step after the "
                         "first 0.5 s")
    ap.add_argument("--ramp", type=int, default=0, metavar="N",
                    help="after the timed steps, idle 1 s and then time N back-to-back steps "
                         "one by one with HIP events; the line gains their mean per range of "
                         "step indices (the clock transient after the GPU idles)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU work budget of the baseline")
    ap.add_argument("--only", choices=["decode", "prefill"], default=None)
    ap.add_argument("--workload", choices=sorted(EXTRA), default=None,
                    help="measure one more workload instead of the headline pair and print its "
                         "own JSON line")
    ap.add_argument("--flush", action="store_true",
                    help="write 512 MB between steps so K/V that fits the 256 MB Infinity Cache "
                         "is read from HBM (kernel timings exclude the flush)")
    ap.add_argument("--linear-vs-vendor", action="store_true",
                    help="time o_proj (nva_linear_forward, the library's own kernels) and "
                         "torch.addmm (hipBLASLt) on the decode and prefill o_proj shapes, one "
                         "JSON line per shape")
    ap.add_argument("--cu-share", type=int, default=0, metavar="K",
                    help="with --workload: run it on a stream limited to K/16 of the CUs "
                         "(hipExtStreamCreateWithCUMask, 2K of the mask's 32 groups of 8 bits), "
                         "for the per-CU bandwidth of a kernel (a mixed step's second stream "
                         "and the graph replays are not limited); the line gains the CU count")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device-to-device copy three times (the "
                         "known-size reference for the FETCH_SIZE/WRITE_SIZE counters)")
    return ap.parse_args()


COPY_BYTES = 1 << 30
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def copy_calibration():
    """Kernels of known HBM traffic for scaling FETCH_SIZE / WRITE_SIZE: a device-to-device copy
    (reads and writes COPY_BYTES) and a read-only sum (reads COPY_BYTES, writes 4 bytes)."""
    import torch
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del dst
    total = None
    for _ in range(3):
        total = src.sum()
    torch.cuda.synchronize()
    log(f"copy calibration: 3 x {COPY_BYTES} bytes device-to-device, 3 x {COPY_BYTES} bytes "
        f"read by a sum ({float(total):.0f})")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE/WRITE_SIZE summary, each
    counter scaled by what it reads for a plain copy of known size; None if not measured."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)[kernel]
        return int(round(t["bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def torch_view(ptr, count, device):
    """A float32 torch tensor over device memory the library owns."""
    import torch

    class _Cai:
        pass

    obj = _Cai()
    obj.__cuda_array_interface__ = {"shape": (count,), "typestr": "<f4",
                                    "data": (ptr, False), "version": 2, "strides": None}
    return torch.as_tensor(obj, device=f"cuda:{device}")


def fill_arena_normal(arena, layer, seed):
    import torch
    k_ptr, v_ptr, nbytes = arena.device_ptrs(layer)
    n = nbytes // 4
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for ptr in (k_ptr, v_ptr):
        t = torch_view(ptr, n, 0)
        chunk = 1 << 28
        for s in range(0, n, chunk):
            t[s:s + chunk].normal_(generator=g)
    torch.cuda.synchronize()


def decode_bytes(wl):
    """Algorithmic bytes of one decode step: K+V rows (per KV head, window-limited), q in,
    out written, block-table entries and context lengths read."""
    kv = wl.kv_bytes_read()
    rows = len(wl.seqs)
    qo = rows * wl.hq * wl.d * 4 * 2
    pages = sum(-(-(c + n) // wl.block_size) for c, n in wl.seqs)
    return kv + qo + 4 * (pages + rows)


def head_norms(wl, seed):
    """Qwen3's per-head q_norm / k_norm (RMSNorm over head_dim, eps 1e-6) with synthetic
    weights near 1."""
    import torch
    from nanollvm_amd import RMSNorm
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    qw = 1.0 + 0.1 * torch.randn(wl.d, device="cuda", generator=g)
    kw = 1.0 + 0.1 * torch.randn(wl.d, device="cuda", generator=g)
    return RMSNorm(qw, 1e-6), RMSNorm(kw, 1e-6)


def kernel_a_bytes(wl, k_out):
    """Algorithmic bytes of the fused norm + RoPE + store kernel: q/k/v read, rotated q (and k)
    written, the rotated k and v rows stored, one cos|sin row, position and slot per token."""
    T, hq, hkv, d = wl.tokens, wl.hq, wl.hkv, wl.d
    return T * (4 * d * (hq + 2 * hkv) + 4 * d * (hq + (hkv if k_out else 0)) +
                4 * d * 2 * hkv + 4 * d + 8)


class cu_masked_stream:
    """A HIP stream restricted to `share`/16 of the device's CUs.  The mask's bits are taken in
    groups of 8 consecutive bits, 2 * share of every 32 groups, spread evenly: each XCD keeps the
    same share of its CUs whether the runtime numbers the bits XCD by XCD or hands consecutive
    bits to the 8 XCDs in turn (with bits i % 16 < share, share 12 ran slower than 8 and share 6
    could not create the stream).  Yields the stream (as a torch ExternalStream) and the number
    of CUs it may use.  The HIP runtime is the one this process already loaded (found in
    /proc/self/maps), so the stream belongs to it."""

    def __init__(self, share):
        if not 1 <= share <= 16:
            raise SystemExit("--cu-share takes 1..16")
        self.share = share

    def __enter__(self):
        import ctypes
        import torch
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise SystemExit("libamdhip64.so is not loaded")
        self.hip = ctypes.CDLL(path)
        n = torch.cuda.get_device_properties(0).multi_processor_count
        words = (n + 31) // 32
        mask = (ctypes.c_uint32 * words)()
        cus = 0
        groups = (n + 7) // 8
        sel = groups * self.share // 16  # groups selected, spread evenly over the mask
        for i in range(n):
            gi = i // 8
            if ((gi + 1) * sel) // groups > (gi * sel) // groups:
                mask[i // 32] |= 1 << (i % 32)
                cus += 1
        self.s = ctypes.c_void_p()
        rc = self.hip.hipExtStreamCreateWithCUMask(ctypes.byref(self.s), ctypes.c_uint32(n), mask)
        if rc != 0:
            raise SystemExit(f"hipExtStreamCreateWithCUMask failed: {rc}")
        return torch.cuda.ExternalStream(self.s.value), cus

    def __exit__(self, *exc):
        import torch
        torch.cuda.synchronize()
        self.hip.hipStreamDestroy(self.s)
        return False


def run_layer(ctx, arena, rope, attn, wl, q, k, v, out_q, out_k, steps, warmup, label,
              flush=None, ramp=0, sustain=0.0):
    import torch
    from nanollvm_amd import Context  # noqa: F401

    ctx.set(**wl.meta.context_args())
    ctx.bind_kv_cache(arena)
    pos = wl.meta.positions
    qn, kn = head_norms(wl, 11)

    def step():
        attn.forward_with_norm_rope(rope, pos, q, k, v, ctx, q_norm=qn, k_norm=kn, q_out=out_q,
                                    k_out=out_k)

    for _ in range(warmup):
        if flush is not None:
            flush()  # also loads the fill kernel before the timed steps
        step()
    # The timed steps run without the library's per-kernel event timing; the same number of
    # steps then runs again with it, for the per-kernel figures.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        if flush is not None:
            flush()
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ctx.reset_stats()
    ctx.set_timing(True)
    torch.cuda.synchronize()
    for _ in range(steps):
        if flush is not None:
            flush()
        step()
    torch.cuda.synchronize()
    ctx.set_timing(False)
    stats = {name: ctx.kernel_stats(name) for name in ("rope_store", "decode", "merge",
                                                       "prefill", "attention")}
    ms = (t1 - t0) * 1e3 / steps
    log(f"{label}: {ms:.4f} ms/step; kernels " + ", ".join(
        f"{n}={s[1] / max(s[0], 1):.4f}ms x{s[0]}" for n, s in stats.items() if s[0]))
    ramp_ms = None
    if ramp > 0:
        ramp_ms = clock_ramp(step, ramp, flush)
        log(f"{label}: per-step ms after 1 s idle: " +
            " ".join(f"[{a}:{b}] {x:.4f}" for a, b, x in ramp_ms))
    sus = None
    if sustain > 0:
        sus = sustained(step, sustain, flush)
        log(f"{label}: sustained {sus}")
    gms = graph_step_ms(ctx, step, steps, flush)
    if gms is not None:
        log(f"{label}: {gms:.4f} ms/step replaying {GRAPH_STEPS} steps per HIP graph")
    plan = time_step_plan(ctx, wl, step)
    plan["graph_ms_per_step"] = None if gms is None else round(gms, 5)
    if ramp_ms is not None:
        plan["ramp"] = ramp_ms
    if sus is not None:
        plan["sustained"] = sus
    return ms, stats, plan


def sustained(step, seconds, flush=None):
    """The step back to back for `seconds` with the board's socket power (W) and gfx clock
    (MHz) sampled every ~10 ms through amdsmi: medians, the power cap and ms/step over the run
    after its first 0.5 s (None for the board figures when amdsmi is unavailable)."""
    import statistics
    import threading
    import torch
    h = cap = None
    try:
        import amdsmi
        amdsmi.amdsmi_init()
        h = amdsmi.amdsmi_get_processor_handles()[0]
        cap = amdsmi.amdsmi_get_power_cap_info(h).get("power_cap")
    except Exception as e:  # no amdsmi module or no access to the board's metrics
        log(f"board power and clock not sampled: {e}")
        h = None
    samples, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            try:
                m = amdsmi.amdsmi_get_gpu_metrics_info(h)
            except Exception:
                return
            samples.append((time.time(), m.get("current_socket_power"), m.get("current_gfxclk")))
            time.sleep(0.01)

    th = threading.Thread(target=sample, daemon=True) if h is not None else None
    torch.cuda.synchronize()
    t = time.perf_counter()
    step()
    torch.cuda.synchronize()
    batch = max(1, int(0.05 / max(time.perf_counter() - t, 1e-5)))
    if th is not None:
        th.start()
    t0 = time.time()
    marks = []
    n = 0
    while time.time() - t0 < seconds:
        for _ in range(batch):
            if flush is not None:
                flush()
            step()
        torch.cuda.synchronize()
        n += batch
        marks.append((time.time(), n))
    stop.set()
    if th is not None:
        th.join()
        try:
            amdsmi.amdsmi_shut_down()
        except Exception:
            pass
    w0 = t0 + 0.5
    first = next((m for m in marks if m[0] >= w0), marks[0])
    last = marks[-1]
    ms = (last[0] - first[0]) * 1e3 / max(last[1] - first[1], 1)
    out = {"seconds": round(last[0] - t0, 2), "steps": last[1], "ms_per_step": round(ms, 5)}
    win = [x for x in samples if first[0] <= x[0] <= last[0]]
    pw = [x[1] for x in win if isinstance(x[1], (int, float))]
    ck = [x[2] for x in win if isinstance(x[2], (int, float))]
    out["socket_power_w"] = statistics.median(pw) if pw else None
    out["gfxclk_mhz"] = statistics.median(ck) if ck else None
    out["power_cap_w"] = round(cap / 1e6) if isinstance(cap, (int, float)) and cap > 0 else None
    out["samples"] = len(win)
    return out


def clock_ramp(step, n, flush=None, idle_s=1.0):
    """Per-step HIP-event times of n back-to-back steps started after idle_s seconds with no GPU
    work: the part drops to a low clock when idle and raises it over the first steps of a
    load.  Returns [first step, end step, mean ms] per range of step indices."""
    import torch
    torch.cuda.synchronize()
    time.sleep(idle_s)
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    for i in range(n):
        ev[i].record(s)
        if flush is not None:
            flush()
        step()
    ev[n].record(s)
    torch.cuda.synchronize()
    d = [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]
    marks = [0, 5, 25, 50, 100, 200, 500, 1000, 2000, 4000, 8000, 16000, 32000]
    out = []
    for a, b in zip(marks, marks[1:]):
        if a >= n:
            break
        b = min(b, n)
        out.append([a, b, round(sum(d[a:b]) / (b - a), 5)])
    return out


GRAPH_STEPS = 10  # layer steps per captured graph


def graph_step_ms(ctx, step, steps, flush=None):
    """The layer step captured GRAPH_STEPS times into one HIP graph (torch.cuda.graph on a side
    stream the context is switched to), as an engine captures the layers of a model step
    together, and the graph replayed until `steps` layer steps have run: wall time per layer
    step, or None when the capture fails.  With --flush each captured step is preceded by the
    flush.  The plan and every buffer already exist from the eager steps, so the captured calls
    launch kernels only."""
    import torch
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        with torch.cuda.stream(s):
            step()
            s.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for _ in range(GRAPH_STEPS):
                    if flush is not None:
                        flush()
                    step()
            s.synchronize()
            g.replay()
            s.synchronize()
            reps = max(1, -(-steps // GRAPH_STEPS))
            t0 = time.perf_counter()
            for _ in range(reps):  # back to back, like the eager steps
                g.replay()
            s.synchronize()
            total = time.perf_counter() - t0
        return total * 1e3 / (reps * GRAPH_STEPS)
    except RuntimeError as e:
        log(f"graph capture failed: {e}")
        return None
    finally:
        torch.cuda.synchronize()
        ctx.set_stream()


def time_step_prepare(ctx, wl, reps=30):
    """Host time of the library's step-metadata producer (Transformer.preparePrefill /
    prepareDecode restated in C++, plus the one upload) for the workload's scheduler state.  The
    nva_seq array is built once, as a Java caller would keep its tables in native memory; the
    timed region is the C call alone."""
    import torch
    from types import SimpleNamespace
    from nanollvm_amd import _native as N
    from nanollvm_amd.step import seq_array
    seqs = [SimpleNamespace(seq_id=b, num_tokens=c + n, num_cached_tokens=c,
                            num_scheduled_tokens=n, block_table=wl.tables[b])
            for b, (c, n) in enumerate(wl.seqs)]
    arr, keep = seq_array(seqs)
    lib = N.load()
    fn = lib.nva_step_prepare_prefill if wl.meta.is_prefill else lib.nva_step_prepare_decode
    assert fn(ctx.handle, arr, len(seqs), wl.block_size) == N.NVA_OK
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn(ctx.handle, arr, len(seqs), wl.block_size)
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    del keep
    m = wl.meta
    tokens = len(m.positions)
    pages = int(sum(len(t) for t in wl.tables))
    bt = m.block_tables.size if m.block_tables is not None else 0
    upload = 4 * (tokens * 2 + bt + 2 * (len(wl.seqs) + 1) + len(wl.seqs))
    return {"build_upload_us": round((t1 - t0) / reps * 1e6, 1), "sequences": len(wl.seqs),
            "tokens": tokens, "pages": pages, "upload_bytes": upload}


def step_metadata(ctx, wl, plan):
    """Per-step host cost: the metadata producer plus one upload, then the first layer's work
    plan (build, upload); the sum is what a scheduler step pays once, before the kernels of its
    first layer."""
    out = time_step_prepare(ctx, wl)
    out.update({k: v for k, v in plan.items()
                if k not in ("graph_ms_per_step", "ramp", "sustained")})
    out["per_step_host_us"] = round(out["build_upload_us"] + plan["plans_per_step"] *
                                    (plan["plan_build_us"] + plan["plan_upload_us"]), 1)
    return out


def time_step_plan(ctx, wl, step, reps=20):
    """Host cost of the work plan a scheduler step builds at its first layer (the library's own
    host timer): after each nva_step_set the first attention call checks every page of the
    step's tables, builds and sorts the work lists and uploads them; later layers reuse the
    plan."""
    import torch
    args = wl.meta.context_args()
    ctx.reset_stats()
    ctx.set_timing(True)
    for _ in range(reps):
        ctx.set(**args)
        step()
        torch.cuda.synchronize()
    ctx.set_timing(False)
    nb, msb = ctx.kernel_stats("plan")
    nu, msu = ctx.kernel_stats("plan_upload")
    ctx.reset_stats()
    build_us = msb / max(nb, 1) * 1e3
    upload_us = msu / max(nu, 1) * 1e3
    return {"plan_build_us": round(build_us, 1), "plan_upload_us": round(upload_us, 1),
            "plans_per_step": round(nb / reps, 2)}


def o_proj_kernel(m, n):
    """The library kernel nva_linear_forward runs for an [m, K] x [n, K]^T o_proj."""
    import torch
    blocks = ((n + 31) // 32) * ((m + 31) // 32)
    blocks16 = ((n + 15) // 16) * ((m + 15) // 16)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if m <= 16:
        return "gemv_kernel (weight-streaming GEMV, <= 16 rows)"
    if 2 * blocks <= cus and 2 * blocks16 >= cus and blocks16 <= 2 * cus:
        return ("skinny16_kernel<8,2> (fp32 MFMA 16x16x4, one 16x16 block per workgroup, "
                "K over 8 waves)")
    if blocks <= cus:
        return "skinny_kernel<8,2> (fp32 MFMA 32x32x2, one 32x32 block per workgroup, K over 8 waves)"
    return "linear_kernel (fp32 MFMA 32x32x2, 128x64 tiles, two workgroups per CU; K slices from a per-CU cost model)"


def time_calls(fn, steps, warmup):
    """ms per call of `steps` back-to-back calls, between two HIP events on torch's current
    stream (the stream the library's context runs on), after `warmup` calls."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_o_proj(ctx, attn_out, wl, steps, warmup, hidden=1024, seed=21):
    """o_proj (Linear.Row, Qwen3-0.6B: [hidden, Hq * d] weight) on this step's attention output,
    timed over back-to-back calls.  Reported beside the step, not inside its value."""
    import torch
    from nanollvm_amd import Linear
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    k = wl.hq * wl.d
    w = torch.randn((hidden, k), device="cuda", generator=g) / math.sqrt(k)
    lin = Linear(w)
    x = attn_out.reshape(attn_out.shape[0], k)
    m = x.shape[0]
    flops = 2.0 * m * hidden * k
    byts = 4.0 * (m * k + hidden * k + m * hidden)
    ms = time_calls(lambda: lin.forward(x, ctx), max(steps, 20), warmup)
    tf = flops / (ms * 1e-3) / 1e12
    return {"kernel": o_proj_kernel(m, hidden), "shape": f"[{m}, {k}] x [{hidden}, {k}]^T",
            "ms": round(ms, 5), "tflops": round(tf, 2),
            "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "gbs": round(byts / (ms * 1e-3) / 1e9, 1)}


# o_proj shapes of Qwen3-0.6B (hidden 1024, Hq * d = 2048): decode batches and the 4096-token
# prefill step; and of the Qwen3-4B-like mixed step (hidden 2560, Hq * d = 4096).
LINEAR_SHAPES = [(1, 2048, 1024), (8, 2048, 1024), (64, 2048, 1024), (128, 2048, 1024),
                 (256, 2048, 1024), (4096, 2048, 1024), (2112, 4096, 2560)]


def linear_vs_vendor(args, ctx):
    """nva_linear_forward against torch.addmm (hipBLASLt) on the same fp32 operands, both timed
    over `steps` back-to-back calls after `warmup`; max-abs error of each against a float64
    product."""
    import torch
    from nanollvm_amd import Linear
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    for m, k, n in LINEAR_SHAPES:
        x = torch.randn((m, k), device="cuda", generator=g)
        w = torch.randn((n, k), device="cuda", generator=g) / math.sqrt(k)
        bias = torch.zeros(n, device="cuda")
        lin = Linear(w)
        ref = x.double() @ w.double().T
        wt = w.T
        res = {}
        for name, fn in (("nva", lambda: lin.forward(x, ctx)),
                         ("hipblaslt", lambda: torch.addmm(bias, x, wt))):
            y = fn()
            ms = time_calls(fn, args.steps, args.warmup)
            res[name] = {"us": round(ms * 1e3, 2), "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 2),
                         "max_abs_vs_f64": float((y.double() - ref).abs().max())}
        print(json.dumps({"shape": f"[{m}, {k}] x [{n}, {k}]^T", "nva_kernel": o_proj_kernel(m, n),
                          **res}), flush=True)


def kernel_a_roofline(wl, stats):
    n, t = stats["rope_store"]
    ms = t / max(n, 1)
    byts = kernel_a_bytes(wl, False)
    gbs = byts / (ms * 1e-3) / 1e9
    return {"kernel": "rope_store_kernel (q/k RMSNorm + RoPE + K/V store)", "bound": "hbm",
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": byts,
            "ms": round(ms, 5)}


def bench_decode(args, ctx):
    import torch
    from nanollvm_amd import Attention, KvCacheArena, RotaryEmbedding
    from nanollvm_amd import workloads as W

    wl = W.qwen3_decode_large()
    log(f"decode workload: {wl.name}: {len(wl.seqs)} rows, {sum(c + n for c, n in wl.seqs)} "
        f"tokens, {wl.num_blocks} blocks")
    arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    fill_arena_normal(arena, 0, 1234)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, wl.max_pos, wl.rope_theta)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    T = wl.tokens
    q = torch.randn((T, wl.hq, wl.d), device="cuda", generator=g)
    k = torch.randn((T, wl.hkv, wl.d), device="cuda", generator=g)
    v = torch.randn((T, wl.hkv, wl.d), device="cuda", generator=g)
    oq = torch.empty_like(q)
    attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
    ms, stats, plan = run_layer(ctx, arena, rope, attn, wl, q, k, v, oq, None, args.steps,
                                args.warmup, "decode", ramp=args.ramp,
                                sustain=args.sustain)
    byts = decode_bytes(wl)
    n_dec, t_dec = stats["decode"]
    dec_ms = t_dec / max(n_dec, 1)
    achieved = byts / (dec_ms * 1e-3) / 1e9
    res = {
        "wl": wl, "ms": ms, "bytes": byts, "gbs": byts / (ms * 1e-3) / 1e9,
        "kernel_ms": {n: s[1] / max(s[0], 1) for n, s in stats.items() if s[0]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("decode"),
                     "kernel": "row_attention_kernel<128,2> (split-KV decode)",
                     "algorithmic_bytes_per_launch": byts},
        "kernel_a": kernel_a_roofline(wl, stats),
        "step_metadata": step_metadata(ctx, wl, plan),
        "graph_ms_per_step": plan["graph_ms_per_step"],
    }
    if "ramp" in plan:
        res["ramp"] = plan["ramp"]
    if "sustained" in plan:
        res["sustained"] = plan["sustained"]
    ctx.set(**wl.meta.context_args())
    ctx.bind_kv_cache(arena)
    res["o_proj"] = time_o_proj(ctx, attn.forward_with_rope(rope, wl.meta.positions, q, k, v, ctx),
                                wl, args.steps, args.warmup)
    rope.close()
    arena.close()
    return res


def bench_prefill(args, ctx):
    import torch
    from nanollvm_amd import Attention, KvCacheArena, RotaryEmbedding
    from nanollvm_amd import workloads as W

    wl = W.qwen3_prefill()
    arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    fill_arena_normal(arena, 0, 99)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, wl.max_pos, wl.rope_theta)
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    T = wl.tokens
    q = torch.randn((T, wl.hq, wl.d), device="cuda", generator=g)
    k = torch.randn((T, wl.hkv, wl.d), device="cuda", generator=g)
    v = torch.randn((T, wl.hkv, wl.d), device="cuda", generator=g)
    oq = torch.empty_like(q)
    attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
    # Paged prefill reads rotated k from the pages, so the rotated k tensor is not requested.
    ms, stats, plan = run_layer(ctx, arena, rope, attn, wl, q, k, v, oq, None, args.steps,
                                args.warmup, "prefill", ramp=args.ramp,
                                sustain=args.sustain)
    flops = 4.0 * wl.d * wl.hq * wl.visible_pairs()
    n_pf, t_pf = stats["prefill"]
    pf_ms = t_pf / max(n_pf, 1)
    achieved = flops / (pf_ms * 1e-3) / 1e12
    res = {
        "workload": wl.name, "ms_per_step": round(ms, 5),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 3),
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "kernel_ms": {n: round(s[1] / max(s[0], 1), 5) for n, s in stats.items() if s[0]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic("prefill"),
                     "kernel": "prefill_kernel<128,2> (fp32 MFMA 16x16x4, 8 waves)",
                     "algorithmic_flops_per_launch": flops},
        "kernel_a": kernel_a_roofline(wl, stats),
        "step_metadata": step_metadata(ctx, wl, plan),
        "graph_ms_per_step": plan["graph_ms_per_step"],
    }
    if "ramp" in plan:
        res["ramp"] = plan["ramp"]
    if "sustained" in plan:
        res["sustained"] = plan["sustained"]
    ctx.set(**wl.meta.context_args())
    ctx.bind_kv_cache(arena)
    res["o_proj"] = time_o_proj(ctx, attn.forward_with_rope(rope, wl.meta.positions, q, k, v, ctx),
                                wl, args.steps, args.warmup)
    rope.close()
    arena.close()
    return res


# Other workloads of the path, measured one per run with --workload (each prints its own line).
def _extra_builders():
    from nanollvm_amd import workloads as W
    return {
        "c1-qwen3-decode-b8": W.qwen3_decode_small,
        "c3-gemma3-decode-local": lambda: W.gemma3_decode(local=True),
        "c3-gemma3-decode-global": lambda: W.gemma3_decode(local=False),
        "c5-qwen3-4b-mixed": W.qwen3_4b_mixed,
        "c5-rows-alone": lambda: W.qwen3_4b_mixed(part="rows"),
        "c5-chunks-alone": lambda: W.qwen3_4b_mixed(part="chunks"),
        "decode-40q-8kv": lambda: W.qwen3_decode_large_heads(40),
        "decode-56q-8kv": lambda: W.qwen3_decode_large_heads(56),
        "gemma4-decode-global": W.gemma4_decode_global,
        "gemma4-decode-global-b256": lambda: W.gemma4_decode_global(batch=256, lo=128,
                                                                     hi=32768),
        "gemma3-prefill-local": lambda: W.gemma3_prefill(local=True),
        "gemma3-prefill-global": lambda: W.gemma3_prefill(local=False),
        "gemma4-prefill-global": W.gemma4_prefill_global,
        "c4-share-head-1of8": lambda: W.qwen3_decode_large_share(8, "head"),
        "c4-share-seq-1of8": lambda: W.qwen3_decode_large_share(8, "seq"),
    }


EXTRA = ["c1-qwen3-decode-b8", "c3-gemma3-decode-local", "c3-gemma3-decode-global",
         "c5-qwen3-4b-mixed", "c5-rows-alone", "c5-chunks-alone", "gemma3-prefill-local",
         "gemma3-prefill-global", "gemma4-prefill-global", "c4-share-head-1of8",
         "c4-share-seq-1of8", "decode-40q-8kv", "decode-56q-8kv", "gemma4-decode-global",
         "gemma4-decode-global-b256"]


def bench_extra(args, ctx):
    """One workload's step: per-kernel times, the decode rows' GB/s over the row kernel, the
    prefill rows' TFLOP/s over the MFMA kernel, and the step's lower bound at peak
    (max of HBM bytes / 8 TB/s and MFMA flops / 157.3 TFLOP/s)."""
    import numpy as np
    import torch
    from nanollvm_amd import Attention, KvCacheArena, RotaryEmbedding

    wl = _extra_builders()[args.workload]()
    log(f"workload: {wl.name}: {len(wl.seqs)} seqs, {wl.tokens} new tokens, {wl.num_blocks} blocks")
    arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    fill_arena_normal(arena, 0, 4321)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, wl.max_pos, wl.rope_theta)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    T = wl.tokens
    q = torch.randn((T, wl.hq, wl.d), device="cuda", generator=g)
    k = torch.randn((T, wl.hkv, wl.d), device="cuda", generator=g)
    v = torch.randn((T, wl.hkv, wl.d), device="cuda", generator=g)
    oq = torch.empty_like(q)
    attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
    junk = torch.empty(512 << 18, device="cuda") if args.flush else None
    flush = (lambda: junk.fill_(1.0)) if args.flush else None
    ms, stats, plan = run_layer(ctx, arena, rope, attn, wl, q, k, v, oq, None, args.steps,
                                args.warmup, wl.name, flush=flush, ramp=args.ramp,
                                sustain=args.sustain)
    dec_rows = [(c, n) for c, n in wl.seqs if n == 1]
    pf_rows = [(c, n) for c, n in wl.seqs if n > 1]
    dec_bytes = 0
    for c, _ in dec_rows:
        vis = min(c + 1, wl.window) if wl.window > 0 else c + 1
        dec_bytes += vis * wl.hkv * wl.d * 8 + wl.hq * wl.d * 8 + 4 * (-(-(c + 1) // wl.block_size) + 1)
    pairs = 0
    for c, n in pf_rows:
        kk = np.arange(c + 1, c + n + 1, dtype=np.int64)
        pairs += int(np.minimum(kk, wl.window).sum() if wl.window > 0 else kk.sum())
    flops = 4.0 * wl.d * wl.hq * pairs
    kms = {n: s[1] / max(s[0], 1) for n, s in stats.items() if s[0]}
    line = {"workload": wl.name, "ms_per_step": round(ms, 5),
            "kernel_ms": {n: round(x, 5) for n, x in kms.items()}, "flush": bool(args.flush),
            "dtype": "f32", "data": "synthetic (seeded N(0,1) q/k/v and pages)"}
    if dec_rows and "decode" in kms:
        gbs = dec_bytes / (kms["decode"] * 1e-3) / 1e9
        line["decode_rows"] = {"rows": len(dec_rows), "bytes": dec_bytes, "gbs": round(gbs, 1),
                               "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if pf_rows and "prefill" in kms:
        tf = flops / (kms["prefill"] * 1e-3) / 1e12
        line["prefill_rows"] = {"tokens": int(sum(n for _, n in pf_rows)), "flops": flops,
                                "tflops": round(tf, 2),
                                "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
    bound = max(dec_bytes / (HBM_PEAK_GBS * 1e9), flops / (FP32_MFMA_PEAK_TFLOPS * 1e12)) * 1e3
    line["lower_bound_ms"] = round(bound, 5)
    line["step_metadata"] = step_metadata(ctx, wl, plan)
    line["attention_ms"] = round(kms.get("attention", 0.0), 5)
    line["graph_ms_per_step"] = plan["graph_ms_per_step"]
    if "ramp" in plan:
        line["ramp"] = plan["ramp"]
    if "sustained" in plan:
        line["sustained"] = plan["sustained"]
    rope.close()
    arena.close()
    return line


def host_cpu():
    """(model string, SIMD lanes of the JDK's FloatVector.SPECIES_PREFERRED on this host:
    16 with AVX-512, 8 with AVX2, 4 otherwise) from /proc/cpuinfo."""
    model, flags, fam = "", set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and not model:
                    model = val
                elif key in ("cpu family", "model", "stepping", "vendor_id") and key not in fam:
                    fam[key] = val
                elif key == "flags" and not flags:
                    flags = set(val.split())
    except OSError:
        pass
    lanes = 16 if "avx512f" in flags else 8 if "avx2" in flags else 4
    simd = "avx512f" if lanes == 16 else "avx2" if lanes == 8 else "sse"
    desc = (f"{model} ({fam.get('vendor_id', '?')} family {fam.get('cpu family', '?')} model "
            f"{fam.get('model', '?')} stepping {fam.get('stepping', '?')}, {simd})")
    return desc, lanes


def cpu_baseline(wl, budget_s):
    """The oracle's Attention.forward (decode branch) on the host cores, over the whole headline
    decode step: the same 256 rows, contexts and block tables (page contents are a tiled
    pattern; values do not change the work).  The oracle is built here for this host
    (-O3 -march=native) and run with the reference's default float kernels, the Vector API
    (FloatKernelsFactory "auto", FloatKernelsFactory.java:41-75) at the host's preferred lane
    count, on every CPU this process may use (availableProcessors, LLM.java:1930-1944) and on
    one thread.  The reference's decode splits each row's head-major jobs over the workers
    (Attention.java:317-325, MatmulRuntime.java:194-225), so at most Hq threads work at once."""
    import tempfile

    import numpy as np
    from oracle import oracle as O

    native = O.build_native(os.path.join(tempfile.mkdtemp(prefix="nva_cpu_"), "liboracle.so"))
    O.set_library(native)
    model, lanes = host_cpu()
    affinity = len(os.sched_getaffinity(0))
    threads = affinity
    m = wl.meta
    shape = (wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    t_fill = time.perf_counter()
    rng = np.random.default_rng(5)
    block = rng.standard_normal(1 << 24, dtype=np.float32)
    kc = np.empty(shape, np.float32)
    vc = np.empty(shape, np.float32)
    for arr, src in ((kc, block), (vc, block[::-1].copy())):
        flat = arr.reshape(-1)
        for s in range(0, flat.size, src.size):
            e = min(flat.size, s + src.size)
            flat[s:e] = src[: e - s]
    rows = len(wl.seqs)
    q = rng.standard_normal((rows, wl.hq, wl.d), dtype=np.float32)
    kv = rng.standard_normal((rows, wl.hkv, wl.d), dtype=np.float32)

    def once(nthreads):
        t0 = time.perf_counter()
        O.attention_forward(wl.hq, wl.d, wl.scale, wl.hkv, is_prefill=False, q=q, k=kv, v=kv,
                            slot_mapping=m.slot_mapping, context_lens=m.context_lens,
                            block_tables=m.block_tables, k_cache=kc, v_cache=vc,
                            threads=nthreads, kernels=lanes)
        return time.perf_counter() - t0

    byts = decode_bytes(wl)
    log(f"cpu baseline: {model}, {affinity} CPUs, {lanes} lanes, whole step "
        f"({byts / 1e9:.2f} GB); pages filled in {time.perf_counter() - t_fill:.1f} s")
    dt1 = once(1)
    reps, spent = 0, 0.0
    while reps == 0 or spent < max(0.0, budget_s - dt1):
        spent += once(threads)
        reps += 1
    dt = spent / reps
    busy = min(threads, wl.hq)
    return {"value": round(byts / dt / 1e9, 3), "unit": "GB/s", "cores": busy,
            "kind": "port",
            "sample": f"the whole decode step ({rows} rows, "
                      f"{int(sum(c + n for c, n in wl.seqs))} context tokens, "
                      f"{byts / 1e9:.2f} GB algorithmic), oracle (C restatement of "
                      f"Attention.attendJobs) built -O3 -march=native on this host, "
                      f"VectorFloatKernels semantics at {lanes} lanes, the reference's "
                      f"head-major job split over {threads} workers (at most {busy} busy: "
                      f"{wl.hq} head jobs per row), mean of {reps} passes of {dt:.3f} s",
            "single_thread": {"value": round(byts / dt1 / 1e9, 3), "seconds": round(dt1, 3)},
            "threads": threads, "nproc": os.cpu_count(), "affinity_cpus": affinity,
            "vector_lanes": lanes, "cpu_model": model}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus above 1 is not "
                                   "supported (the path shards by sequence or KV head with no "
                                   "exchange, but only the one-GPU kernel is built)"}))
        sys.exit(2)
    import torch
    from nanollvm_amd import Context

    torch.cuda.init()
    ctx = Context(0)
    if args.linear_vs_vendor:
        linear_vs_vendor(args, ctx)
        ctx.close()
        return
    if args.workload:
        if args.cu_share:
            with cu_masked_stream(args.cu_share) as (ext, cus):
                with torch.cuda.stream(ext):
                    ctx.set_stream(ext)
                    line = bench_extra(args, ctx)
                    torch.cuda.synchronize()
                    ctx.set_stream()
            line["cu_share"] = {"sixteenths": args.cu_share, "cus": cus}
            if "decode_rows" in line:
                line["cu_share"]["decode_gbs_per_cu"] = round(line["decode_rows"]["gbs"] / cus, 2)
        else:
            line = bench_extra(args, ctx)
        ctx.close()
        print(json.dumps(line), flush=True)
        return
    dec = pf = None
    if args.only in (None, "decode"):
        dec = bench_decode(args, ctx)
    if args.only in (None, "prefill"):
        pf = bench_prefill(args, ctx)
    ctx.close()
    if args.copy_calibration:
        copy_calibration()
    cpu = None
    if dec is not None and not args.no_cpu:
        cpu = cpu_baseline(dec["wl"], args.cpu_seconds)
    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded N(0,1) q/k/v and pages; seeded block tables)"}
    if dec is not None:
        wl = dec["wl"]
        line.update({
            "value": round(dec["gbs"], 1), "unit": "GB/s", "ms_per_step": round(dec["ms"], 5),
            "config": {"workload": wl.name, "q_heads": wl.hq, "kv_heads": wl.hkv,
                       "head_dim": wl.d, "block_size": wl.block_size, "rows": len(wl.seqs),
                       "context_tokens": int(sum(c + n for c, n in wl.seqs)),
                       "kv_bytes_per_step": wl.kv_bytes_read(),
                       "step": "fused RoPE+store, split-KV decode, merge"},
            "tokens_per_s_per_layer": round(len(wl.seqs) / (dec["ms"] * 1e-3), 1),
            "kernel_ms": {n: round(x, 5) for n, x in dec["kernel_ms"].items()},
            "roofline": dec["roofline"],
            "kernel_a": dec["kernel_a"],
            "step_metadata": dec["step_metadata"],
            "graph_ms_per_step": dec["graph_ms_per_step"],
            "o_proj": dec["o_proj"],
        })
        if "ramp" in dec:
            line["ramp"] = dec["ramp"]
        if "sustained" in dec:
            line["sustained"] = dec["sustained"]
    else:
        line.update({"value": pf["tflops"], "unit": "TFLOP/s", "ms_per_step": pf["ms_per_step"],
                     "config": {"workload": pf["workload"]}, "roofline": pf["roofline"]})
    if pf is not None:
        line["prefill"] = pf
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
