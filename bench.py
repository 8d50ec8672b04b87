"""Benchmark of the Magnetar MI355X Provider's hot path on one GPU.

Prints ONE JSON line. The headline (`value`) is the workload BASELINE.json's
metric is quoted on that fits one GPU: configs[1], the f32 matmul, at
4096^3 (the north star's MFMA target). The same run measures every other
hot-path Kernel at its BASELINE shape (`kernels`), each as algorithmic
GB/s or TFLOP/s over the average launch time from HIP events recorded on
the library's own stream, and as a fraction of the MI355X roofline.
Inputs are resident in HBM before timing starts. The CPU oracle is timed on
a bounded sample of the headline workload on this host (`cpu_baseline`), and
beside every other kernel on a bounded sample of its workload
(`kernels.<name>.cpu`).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "magnetar-provider-cuda_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
METRIC = "per-kernel GB/s or TFLOP/s (% roofline); decoder-block tokens/s, 1 MI355X"
MB = 1e6
HEADLINE = "matmul_4096"
# HBM bytes per launch measured with rocprofv3 (FETCH_SIZE + WRITE_SIZE,
# scaled by a plain copy's reading); null until measured.
TRAFFIC: dict = {"matmul_4096": 470_768_640}  # profiles/matmul_4096_mfma_gemm.md


# Untimed GPU time each case runs before its warm-up and timed launches.
PREHEAT_S = 0.1


def seed(config: int, tensor: int) -> int:
    return 0x4D414732 ^ (config << 16) ^ tensor


class Case:
    """One kernel at one shape: `launch()` enqueues exactly one call.
    `tokens`, when set, also reports tokens/s (the decoder-block chains)."""

    def __init__(self, name, launch, work, bound, shape, tokens=None):
        self.name, self.launch, self.work, self.bound, self.shape = name, launch, work, bound, shape
        self.tokens = tokens

    def measure(self, dev, steps, warmup, preheat_s=PREHEAT_S):
        # The MI355X raises its clock over tens of milliseconds of sustained
        # load (2.06 -> 2.38 GHz measured on the GEMM with s_memtime against
        # s_memrealtime), so each case first runs its own launches, untimed,
        # for `preheat_s` of GPU time; then the W warm-up launches, then
        # exactly `steps` timed ones.
        spent, i = 0.0, 0
        while spent < preheat_s:
            dev.timer_start()
            for _ in range(4):
                self.launch(i)
                i += 1
            spent += dev.timer_stop() * 1e-3
        for i in range(warmup):
            self.launch(i)
        dev.sync()
        # A case whose `steps` launches take under 5 ms (launch-bound ones
        # such as the C1 block) is timed over 5 such windows and the median
        # window counts, to damp the noise of one short window. Every window
        # times exactly `steps` launches between synchronisations.
        # The host's own time to enqueue a launch (the calls return before
        # the GPU finishes) is kept beside it: what a host loop pays per call.
        times, host = [], []
        while not times or (times[0] * steps < 5.0 and len(times) < 5):
            dev.timer_start()
            t0 = time.perf_counter()
            for j in range(steps):
                self.launch(warmup + len(times) * steps + j)
            host.append((time.perf_counter() - t0) / steps)
            times.append(dev.timer_stop() / steps)
        windows = len(times)
        ms = sorted(times)[windows // 2]
        host_us = sorted(host)[windows // 2] * 1e6
        if self.bound == "hbm":
            achieved = self.work / (ms * 1e-3) / 1e9
            peak, unit = HBM_PEAK_GBS, "GB/s"
        else:
            achieved = self.work / (ms * 1e-3) / 1e12
            peak, unit = FP32_MFMA_PEAK_TFLOPS, "TFLOP/s"
        out = {"ms": ms, "achieved": achieved, "unit": unit, "peak": peak,
               "frac": achieved / peak, "work": self.work, "bound": self.bound,
               "shape": self.shape, "windows": windows, "host_us": round(host_us, 2)}
        if self.tokens:
            out["tokens_per_s"] = self.tokens / (ms * 1e-3)
        return out


# MI355X's 256 MB Infinity Cache would hold a whole working set of the
# bandwidth cases between repeated launches; each such case cycles through
# enough copies of its tensors (>= 1 GB) that every launch reads and writes
# HBM, as a single pass over fresh data does.
CACHE_ROTATION_BYTES = 1 << 30


def _copies(footprint):
    return max(1, -(-CACHE_ROTATION_BYTES // footprint))


def streaming_cases(dev, orc):
    from magnetar_hip import ops, MHIP_F16, MHIP_BF16
    cases = []
    rows, cols = 8192, 4096
    n = rows * cols
    f32 = 4
    r3, r2 = _copies(3 * n * f32), _copies(2 * n * f32)
    xs = [dev.upload(orc.normal(n, seed(3, 10 + i))) for i in range(max(r3, r2))]
    ys = [dev.upload(orc.normal(n, seed(3, 20 + i))) for i in range(r3)]
    outs = [dev.empty((n,)) for _ in range(max(r3, r2))]
    gain = dev.upload(orc.normal(cols, seed(3, 2), 1.0, 0.1))
    cases.append(Case("add", lambda i: ops.add(dev, xs[i % r3], ys[i % r3], outs[i % r3]),
                      3 * n * f32, "hbm", [n]))
    cases.append(Case("mul", lambda i: ops.mul(dev, xs[i % r3], ys[i % r3], outs[i % r3]),
                      3 * n * f32, "hbm", [n]))
    cases.append(Case("residual_add", lambda i: ops.add(dev, xs[i % r3], ys[i % r3], outs[i % r3]),
                      3 * n * f32, "hbm", [n]))
    cases.append(Case("silu", lambda i: ops.silu(dev, xs[i % r2], outs[i % r2]), 2 * n * f32,
                      "hbm", [n]))
    cases.append(Case("silu_mul", lambda i: ops.silu_mul(dev, xs[i % r3], ys[i % r3], outs[i % r3]),
                      3 * n * f32, "hbm", [n]))
    x2 = [_reshape(x, (rows, cols)) for x in xs]
    o2 = [_reshape(o, (rows, cols)) for o in outs]
    cases.append(Case("rmsnorm", lambda i: ops.rmsnorm(dev, x2[i % r2], gain, 1e-5, out=o2[i % r2]),
                      2 * n * f32 + cols * f32, "hbm", [rows, cols]))
    sm = [dev.upload(orc.normal(n, seed(3, 30 + i), 0.0, 2.0).reshape(rows, cols)) for i in range(r2)]
    cases.append(Case("softmax", lambda i: ops.softmax_rows(dev, sm[i % r2], out=o2[i % r2]),
                      2 * n * f32, "hbm", [rows, cols]))
    rp = ops.rope_params(128, 32)
    cases.append(Case("rope", lambda i: ops.rope(dev, x2[i % r2], rp, out=o2[i % r2]), 2 * n * f32,
                      "hbm", [rows, 32 * 128]))
    # Embedding: 8192 ids into a [128000, 4096] table (2.1 GB resident).
    vocab = 128000
    table = dev.empty((vocab, cols))
    _fill_normal(dev, table, seed(3, 4))
    re = _copies(2 * 8192 * cols * f32)
    ids = [dev.upload(orc.token_ids(8192, seed(3, 50 + i), vocab)) for i in range(re)]
    emb_out = [dev.empty((8192, cols)) for _ in range(re)]
    cases.append(Case("embedding", lambda i: ops.embedding(dev, table, ids[i % re], emb_out[i % re]),
                      2 * 8192 * cols * f32 + 8192 * f32, "hbm", [8192, cols]))
    # Half path: 64M elements per tensor.
    hn = 1 << 26
    rh = _copies(3 * hn * 2)
    for dname, dt in (("f16", MHIP_F16), ("bf16", MHIP_BF16)):
        ha = [dev.upload(orc.encode_half(orc.normal(hn, seed(3, 60 + i)), dt), half=dt) for i in range(rh)]
        hb = [dev.upload(orc.encode_half(orc.normal(hn, seed(3, 70 + i)), dt), half=dt) for i in range(rh)]
        ho = [dev.empty((hn,), np.uint16, dt) for _ in range(rh)]
        for op in ("add", "mul"):
            cases.append(Case(f"{op}_{dname}",
                              (lambda i, ha=ha, hb=hb, ho=ho, op=op, dt=dt:
                               ops.half_binary(dev, ha[i % rh], hb[i % rh], op, dt, ho[i % rh])),
                              3 * hn * 2, "hbm", [hn]))
    return cases


def calibration_cases(dev, orc):
    """A plain copy of known size (scale by 1.0 over 64M floats: 268 MB read,
    268 MB written), run only when named: it calibrates the rocprofv3
    FETCH_SIZE / WRITE_SIZE counters against bytes that are known."""
    from magnetar_hip import ops
    n = 1 << 26
    x = dev.upload(orc.normal(n, seed(9, 0)))
    y = dev.empty((n,))
    return [Case("calibration_copy", lambda i: ops.scale(dev, x, 1.0, y), 2 * n * 4, "hbm", [n])]


def matmul_cases(dev, orc):
    from magnetar_hip import ops
    cases = []
    for size in (1024, 2048, 4096, 8192):
        a = dev.upload(orc.uniform(size * size, seed(2, size), -1.0, 1.0).reshape(size, size))
        b = dev.upload(orc.uniform(size * size, seed(2, size + 1), -1.0, 1.0).reshape(size, size))
        c = dev.empty((size, size))
        cases.append(Case(f"matmul_{size}", (lambda i, a=a, b=b, c=c: ops.matmul(dev, a, b, out=c)),
                          2.0 * size ** 3, "mfma", [size, size, size]))
    a = dev.upload(orc.uniform(4096, seed(2, 1), -1.0, 1.0).reshape(1, 4096))
    rb = _copies(4096 * 11008 * 4)
    bs = [dev.upload(orc.uniform(4096 * 11008, seed(2, 2 + i), -1.0, 1.0).reshape(4096, 11008))
          for i in range(rb)]
    c = dev.empty((1, 11008))
    cases.append(Case("matmul_1x4096x11008", lambda i: ops.matmul(dev, a, bs[i % rb], out=c),
                      4 * (4096 * 11008 + 4096 + 11008), "hbm", [1, 4096, 11008]))
    # The same product over a compact weight (bf16 bits, widened exactly).
    rh = _copies(4096 * 11008 * 2)
    hs = [_device_normal(dev, (4096, 11008), seed(2, 40 + i), 0.5, bf16=True) for i in range(rh)]
    cases.append(Case("matmul_1x4096x11008_bf16w",
                      lambda i: ops.matmul_bf16w(dev, a, hs[i % rh], out=c),
                      2 * 4096 * 11008 + 4 * (4096 + 11008), "hbm", [1, 4096, 11008]))
    return cases


def attention_cases(dev, orc):
    from magnetar_hip import ops
    cases = []
    B, S, H, d = 4, 2048, 32, 128
    q = dev.upload(orc.normal(B * S * H * d, seed(4, 0)).reshape(B * S, H * d))
    k = dev.upload(orc.normal(B * S * H * d, seed(4, 1)).reshape(B * S, H * d))
    v = dev.upload(orc.normal(B * S * H * d, seed(4, 2)).reshape(B * S, H * d))
    o = dev.empty((B * S, H * d))
    p = ops.attention_params(S, S, H, d, causal=True, batch=B)
    flops = 4.0 * d * S * (S + 1) / 2 * B * H
    cases.append(Case("attention_prefill", lambda i: ops.attention(dev, q, k, v, p, o), flops,
                      "mfma", [B, H, S, d]))
    B2, KV = 8, 4096
    q2 = dev.upload(orc.normal(B2 * H * d, seed(4, 3)).reshape(B2, H * d))
    k2 = dev.empty((B2 * KV, H * d))
    v2 = dev.empty((B2 * KV, H * d))
    _fill_normal(dev, k2, seed(4, 4))
    _fill_normal(dev, v2, seed(4, 5))
    o2 = dev.empty((B2, H * d))
    p2 = ops.attention_params(1, KV, H, d, causal=True, batch=B2)
    nbytes = 2 * B2 * KV * H * d * 4 + 2 * B2 * H * d * 4
    cases.append(Case("attention_decode", lambda i: ops.attention(dev, q2, k2, v2, p2, o2), nbytes,
                      "hbm", [B2, H, KV, d]))
    return cases


def _device_normal(dev, shape, s, std, bf16=False):
    """A seeded N(0, std) device tensor, generated on the host in chunks; with
    `bf16`, stored as bf16 bit patterns (the f32 values truncated)."""
    import ctypes
    from oracle import oracle as orc
    from magnetar_hip._lib import call
    arr = dev.empty(shape, np.uint16 if bf16 else np.float32)
    n = int(np.prod(shape))
    size = 2 if bf16 else 4
    chunk = 16 << 20
    for i0 in range(0, n, chunk):
        host = orc.normal(min(chunk, n - i0), s + i0, 0.0, std)
        if bf16:
            host = (host.view(np.uint32) >> 16).astype(np.uint16)
        call("mhip_upload", dev.ctx, ctypes.c_void_p(arr.ptr + size * i0),
             host.ctypes.data_as(ctypes.c_void_p), host.nbytes)
    return arr


def selection_cases(dev, orc):
    """Two decode-step helpers: greedy selection over a Llama-2 vocabulary
    row and one K/V row appended in place (kv-write). Both are launch-bound;
    their bytes are reported for completeness. Greedy selection returns its
    column to the host (as the reference does), so each call's time includes
    that 8-byte download and its synchronisation."""
    from magnetar_hip import ops
    cases = []
    vocab = 32000
    logits = dev.upload(orc.normal(vocab, seed(5, 40)).reshape(1, vocab))
    cases.append(Case("greedy_select_32000", lambda i: ops.greedy_select(dev, logits, 0),
                      vocab * 4, "hbm", [1, vocab]))
    width, capacity = 4096, 2048
    store = dev.empty((capacity, width))
    row = dev.upload(orc.normal(width, seed(5, 41)).reshape(1, width))
    cases.append(Case("kv_write_1x4096", lambda i: ops.kv_write(dev, store, row, i % capacity),
                      2 * width * 4, "hbm", [1, width]))
    return cases


def decoder_cases(dev, orc, graphs=True):
    """The chained decoder block: config 0 (tiny, seq 32) and config 4
    (Llama-2-7B shapes: prefill 512, decode one token at KV 2048)."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    cases = []

    def block(shapes, cfg, cache_rows, max_seq, bf16=False):
        w = {}
        for i, (name, shape) in enumerate(shapes.weight_shapes().items()):
            if name.endswith("norm"):
                w[name] = dev.upload(np.ones(shape, np.float32))
            else:
                w[name] = _device_normal(dev, shape, seed(cfg, 16 + i), 0.02, bf16=bf16)
        return DecoderBlock(dev, shapes, w, cache_rows=cache_rows, max_seq=max_seq,
                            bf16_weights=bf16)

    tiny = Shapes(vocab=1024, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=688)
    b0 = block(tiny, 0, 32, 32)
    ids0 = dev.upload(orc.token_ids(32, seed(0, 1), 1024))
    out0 = dev.empty((32, 256))
    w0 = 4 * (4 * 256 * 256 + 3 * 256 * 688)
    cases.append(Case("decoder_c1_seq32", lambda i: b0.forward(ids0, 0, out0), w0, "hbm",
                      [32, 256], tokens=32))
    # The same block captured once as a HIP graph and replayed (launch-bound).
    if graphs:
        b0.forward(ids0, 0, out0)
        dev.capture_begin(0)
        b0.forward(ids0, 0, out0)
        g0 = dev.capture_end()
        cases.append(Case("decoder_c1_seq32_graph", lambda i: g0.launch(0), w0, "hbm", [32, 256],
                          tokens=32))
    big = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    b4 = block(big, 4, 2049, 512)
    ids_p = dev.upload(orc.token_ids(512, seed(4, 8), 32000))
    out_p = dev.empty((512, 4096))
    flops = 2.0 * 512 * (4 * 4096 * 4096 + 3 * 4096 * 11008) + 4.0 * 128 * 512 * 513 / 2 * 32
    cases.append(Case("decoder_c5_prefill512", lambda i: b4.forward(ids_p, 0, out_p), flops, "mfma",
                      [512, 4096], tokens=512))
    ids_d = dev.upload(orc.token_ids(1, seed(4, 9), 32000))
    out_d = dev.empty((1, 4096))
    weight_bytes = 4 * (4 * 4096 * 4096 + 3 * 4096 * 11008)
    kv_bytes = 2 * 2049 * 4096 * 4
    cases.append(Case("decoder_c5_decode_kv2048", lambda i: b4.forward(ids_d, 2048, out_d),
                      weight_bytes + kv_bytes, "hbm", [1, 4096], tokens=1))
    # A decode step captured with position, cache row and key count advancing
    # (here at the last cache row, so replays run at offset 0).
    from magnetar_hip.device import ADVANCE_KEY_COUNT, ADVANCE_POSITION_OFFSET, ADVANCE_ROW_OFFSET
    if graphs:
        b4.forward(ids_d, 2048, out_d)
        dev.capture_begin(ADVANCE_POSITION_OFFSET | ADVANCE_KEY_COUNT | ADVANCE_ROW_OFFSET)
        b4.forward(ids_d, 2048, out_d)
        g4 = dev.capture_end()
        cases.append(Case("decoder_c5_decode_kv2048_graph", lambda i: g4.launch(0),
                          weight_bytes + kv_bytes, "hbm", [1, 4096], tokens=1))
    # Config 4 decode with compact bf16 weights (a bf16 checkpoint): half the
    # weight bytes, the same f32 arithmetic.
    b4h = block(big, 4, 2049, 1, bf16=True)
    cases.append(Case("decoder_c5_decode_kv2048_bf16w", lambda i: b4h.forward(ids_d, 2048, out_d),
                      weight_bytes // 2 + kv_bytes, "hbm", [1, 4096], tokens=1))
    return cases


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_threads() -> int:
    """Threads this process may use: its CPU affinity, capped by
    OMP_NUM_THREADS where the host sets a share."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() and int(cap) > 0 else n


def cpu_baseline(orc, runs=5, run_s=1.5):
    """The oracle's matmul (f32, k ascending; oracle/oracle.c orc_matmul_rows)
    on whole rows of the 4096^3 headline product: median of `runs` timed runs
    after a warm-up, single-threaded (the reference order) and parallel over
    rows on every usable host thread (ctypes releases the GIL). Each run
    covers as many rows as take about `run_s` seconds on one thread."""
    from concurrent.futures import ThreadPoolExecutor
    size = 4096
    a = orc.uniform(size * size, seed(2, size), -1.0, 1.0).reshape(size, size)
    b = orc.uniform(size * size, seed(2, size + 1), -1.0, 1.0).reshape(size, size)
    t0 = time.perf_counter()
    orc.matmul_rows(a, b, 0, 2)  # warm-up, and the per-row time
    per_row = (time.perf_counter() - t0) / 2
    rows = int(min(size, max(2, run_s / max(per_row, 1e-6))))
    flop_per_row = 2.0 * size * size

    def timed(fn):
        times = []
        for _ in range(runs):
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
        return float(np.median(times))

    single = timed(lambda: orc.matmul_rows(a, b, 0, rows))
    threads = _host_threads()
    par_rows = min(size, rows * threads)
    bounds = np.linspace(0, par_rows, threads + 1).astype(int)
    with ThreadPoolExecutor(threads) as pool:
        def parallel():
            list(pool.map(lambda i: orc.matmul_rows(a, b, int(bounds[i]), int(bounds[i + 1])),
                          range(threads)))
        parallel()  # warm-up
        par = timed(parallel)
    single_tflops = flop_per_row * rows / single / 1e12
    return {"value": round(flop_per_row * par_rows / par / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"{par_rows} of {size} rows of the {size}^3 f32 product split over {threads} "
                      f"threads, median of {runs} runs ({par:.2f} s each) after a warm-up "
                      f"(oracle/oracle.c orc_matmul_rows)",
            "single_thread": {"value": round(single_tflops, 6), "cores": 1,
                              "sample": f"{rows} rows, median of {runs} runs ({single:.2f} s each)"},
            "cpu_model": _cpu_model(), "nproc": os.cpu_count()}


# ---------------------------------------------------------------------------
# Per-kernel CPU legs: the oracle (oracle/oracle.c, the reference CPU
# Provider's arithmetic) timed beside every kernel on a bounded sample of the
# same workload, on this host. Reported baselines only.
# ---------------------------------------------------------------------------

class CpuLeg:
    """`run(r0, r1)` does units [r0, r1) of a case's workload on the oracle
    (rows, heads, rows of a product, whole block calls); `units` is the
    workload's count and `data_units` how many the host sample holds; `work`
    is the GPU case's algorithmic bytes or flops per unit and `tokens` its
    tokens per unit. `split`: units are divided over host threads; otherwise
    one call runs them (`cores` then says how many threads that call uses).
    `single`: a run(r0, r1) for the single-thread figure where `run` itself
    uses several threads (the C5 prefill block's split products)."""

    def __init__(self, run, units, work, what, data_units=None, tokens=0.0, split=True, cores=1,
                 single=None, single_what=None, single_work=0.0, single_tokens=0.0):
        self.run, self.units, self.work, self.what = run, units, work, what
        self.data_units = data_units or units
        self.tokens, self.split, self.cores = tokens, split, cores
        self.single, self.single_what = single, single_what
        self.single_work, self.single_tokens = single_work, single_tokens


def _timed_units(run, n, units, runs, pool):
    """Median seconds of `runs` passes over `units` units split over `n`
    threads (one call when n is 1), after one untimed pass."""
    bounds = np.linspace(0, units, n + 1).astype(int)

    def once():
        if n == 1:
            run(0, units)
        else:
            list(pool.map(lambda i: run(int(bounds[i]), int(bounds[i + 1])), range(n)))
    once()
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        once()
        times.append(time.perf_counter() - t)
    return float(np.median(times))


def time_cpu_leg(leg, bound, threads, target_s=0.4, runs=3):
    """The oracle on a bounded sample of the case's workload, two ways
    on every usable host thread ("value", "cores")
    and on one thread ("single_thread"). A split leg divides units over
    threads; a leg that is one sequential call (a GEMV, a decode step, a
    selection) runs that many independent calls at once for its all-core
    figure (throughput of concurrent calls over the same data)."""
    from concurrent.futures import ThreadPoolExecutor
    t = time.perf_counter()
    leg.run(0, 1)  # warm-up, and the time of one unit
    per_unit = max(time.perf_counter() - t, 1e-7)
    scale = 1e9 if bound == "hbm" else 1e12
    unit = "GB/s" if bound == "hbm" else "TFLOP/s"

    def figure(units, sec, cores, sample):
        out = {"value": round(leg.work * units / sec / scale, 6), "unit": unit, "cores": cores,
               "sample": sample + f", median of {runs} runs ({sec * 1e3:.1f} ms each) after a warm-up"}
        if leg.tokens:
            out["tokens_per_s"] = round(leg.tokens * units / sec, 2)
        return out

    with ThreadPoolExecutor(max(1, threads)) as pool:
        if leg.split:
            n = min(threads, leg.data_units)
            units = int(min(leg.data_units, max(n, target_s * n / per_unit)))
            sec = _timed_units(leg.run, n, units, runs, pool)
            out = figure(units, sec, n, f"{units} of {leg.units} {leg.what} over {n} threads")
            units1 = int(min(leg.data_units, max(1, target_s / 2 / per_unit)))
            sec1 = _timed_units(leg.run, 1, units1, runs, pool)
            out["single_thread"] = figure(units1, sec1, 1, f"{units1} of {leg.units} {leg.what}")
        else:
            # One call holds `units` units in sequence.
            units = int(min(100000, max(1, target_s / per_unit)))
            if leg.cores > 1:
                sec = _timed_units(leg.run, 1, units, runs, pool)
                out = figure(units, sec, leg.cores, f"{units} {leg.what}")
                if leg.single is not None:
                    t = time.perf_counter()
                    leg.single(0, 1)
                    per1 = max(time.perf_counter() - t, 1e-7)
                    units1 = int(min(100000, max(1, target_s / 2 / per1)))
                    sec1 = _timed_units(leg.single, 1, units1, runs, pool)
                    single = figure(units1, sec1, 1, f"{units1} {leg.single_what}")
                    single["value"] = round(leg.single_work * units1 / sec1 / scale, 6)
                    if leg.tokens:
                        single["tokens_per_s"] = round(leg.single_tokens * units1 / sec1, 2)
                    out["single_thread"] = single
            else:
                sec1 = _timed_units(leg.run, 1, units, runs, pool)
                single = figure(units, sec1, 1, f"{units} {leg.what}")
                n = threads
                # n independent calls at once, each `units` long.
                sec = _timed_units(lambda a, b: leg.run(0, units), n, n, runs, pool)
                out = figure(units * n, sec, n,
                             f"{n} concurrent calls of {units} {leg.what} (independent, over "
                             f"the same host data)")
                out["single_thread"] = single
    out["kind"] = "port"
    return out


def cpu_legs(orc, names):
    """CpuLeg per bench case name (only those in `names`). Inputs are host
    samples of each case's shape; their values (numpy's generator, same
    distributions) do not change the oracle's time."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from reference_chain import host_threads, reference_block
    from magnetar_hip.decoder import Shapes
    rng = np.random.default_rng(7)
    normal = lambda shape, std=1.0, mean=0.0: (rng.standard_normal(shape, np.float32) * std + mean)
    legs = {}
    want = lambda *ns: any(n in names for n in ns)
    rows, cols = 8192, 4096
    row_bytes = cols * 4
    if want("add", "mul", "residual_add", "silu", "silu_mul", "rmsnorm", "softmax", "rope"):
        x, y = normal((rows, cols)), normal((rows, cols))
        sm = x * np.float32(2.0)
        gain = normal(cols, 0.1, 1.0)
        what = "rows of [8192, 4096]"
        legs["add"] = CpuLeg(lambda a, b: orc.add(x[a:b], y[a:b]), rows, 3 * row_bytes, what)
        legs["mul"] = CpuLeg(lambda a, b: orc.mul(x[a:b], y[a:b]), rows, 3 * row_bytes, what)
        legs["residual_add"] = legs["add"]
        legs["silu"] = CpuLeg(lambda a, b: orc.silu(x[a:b]), rows, 2 * row_bytes, what)
        legs["silu_mul"] = CpuLeg(lambda a, b: orc.silu_mul(x[a:b], y[a:b]), rows, 3 * row_bytes, what)
        legs["rmsnorm"] = CpuLeg(lambda a, b: orc.rmsnorm(x[a:b], gain, 1e-5), rows,
                                 2 * row_bytes, what)
        legs["softmax"] = CpuLeg(lambda a, b: orc.softmax_rows(sm[a:b]), rows, 2 * row_bytes, what)
        legs["rope"] = CpuLeg(lambda a, b: orc.rope(x[a:b], orc.rope_params(128, 32, position_offset=a)),
                              rows, 2 * row_bytes, what)
    if want("embedding"):
        vocab = 16384  # a 268 MB slice of the 128000-row table: gathers stay DRAM reads
        table = normal((vocab, cols))
        ids = rng.integers(0, vocab, 8192).astype(np.float32)
        legs["embedding"] = CpuLeg(lambda a, b: orc.embedding(table, ids[a:b]), 8192,
                                   2 * row_bytes + 4, "ids into a [16384, 4096] table")
    for dname, dt in (("f16", 0), ("bf16", 1)):
        if want(f"add_{dname}", f"mul_{dname}"):
            ha = orc.encode_half(normal((4096, 4096)), dt)
            hb = orc.encode_half(normal((4096, 4096)), dt)
            for op in ("add", "mul"):
                legs[f"{op}_{dname}"] = CpuLeg(
                    (lambda a, b, ha=ha, hb=hb, op=op, dt=dt: orc.half_binary(ha[a:b], hb[a:b], dt, op)),
                    16384, 3 * 4096 * 2, "rows of 4096 of the 64M-element tensors", data_units=4096)
    for size in (1024, 2048, 4096, 8192):
        if want(f"matmul_{size}"):
            a_m, b_m = normal((size, size)), normal((size, size))
            legs[f"matmul_{size}"] = CpuLeg(
                (lambda r0, r1, a_m=a_m, b_m=b_m: orc.matmul_rows(a_m, b_m, r0, r1)), size,
                2.0 * size * size, f"rows of the {size}^3 product")
    if want("matmul_1x4096x11008", "matmul_1x4096x11008_bf16w"):
        a1, b1 = normal((1, 4096)), normal((4096, 11008))
        gemv = lambda r0, r1: [orc.matmul_rows(a1, b1, 0, 1) for _ in range(r0, r1)]
        legs["matmul_1x4096x11008"] = CpuLeg(gemv, 1, 4 * (4096 * 11008 + 4096 + 11008),
                                             "whole products in a row", split=False)
        legs["matmul_1x4096x11008_bf16w"] = CpuLeg(gemv, 1, 2 * 4096 * 11008 + 4 * (4096 + 11008),
                                                   "whole products in a row (over the widened f32 "
                                                   "weight)", split=False)
    if want("attention_prefill"):
        S, H, d = 2048, 32, 128
        q, k, v = normal((S, H * d)), normal((S, H * d)), normal((S, H * d))
        ap = orc.attention_params(S, S, H, d, causal=True)
        legs["attention_prefill"] = CpuLeg(lambda a, b: orc.attention(q, k, v, ap, heads=(a, b)),
                                           4 * H, 4.0 * d * S * (S + 1) / 2,
                                           "(batch, head) pairs of B4 H32 S2048 d128", data_units=H)
    if want("attention_decode"):
        KV, H, d = 4096, 32, 128
        q, k, v = normal((1, H * d)), normal((KV, H * d)), normal((KV, H * d))
        ad = orc.attention_params(1, KV, H, d, causal=True)
        legs["attention_decode"] = CpuLeg(lambda a, b: orc.attention(q, k, v, ad, heads=(a, b)),
                                          8 * H, 2 * KV * d * 4 + 2 * d * 4,
                                          "(batch, head) pairs of B8 H32 KV4096 d128", data_units=H)
    if want("greedy_select_32000"):
        logits = normal(32000)
        legs["greedy_select_32000"] = CpuLeg(
            lambda a, b: [orc.greedy_select(logits) for _ in range(a, b)], 1, 32000 * 4,
            "selections over a 32000-column row", split=False)
    if want("kv_write_1x4096"):
        store, row = np.zeros((2048, 4096), np.float32), normal(4096)

        def kv(a, b):
            for r in range(a, b):
                store[r % 2048] = row
        legs["kv_write_1x4096"] = CpuLeg(kv, 2048, 2 * 4096 * 4,
                                         "row appends into a [2048, 4096] store (numpy copy)",
                                         split=False)
    if want("decoder_c1_seq32", "decoder_c1_seq32_graph"):
        tiny = Shapes(vocab=1024, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=688)
        wt = {n: (np.ones(sh, np.float32) if n.endswith("norm") else normal(sh, 0.02))
              for n, sh in tiny.weight_shapes().items()}
        ids0 = rng.integers(0, 1024, 32).astype(np.float32)
        z = np.zeros((32, 256), np.float32)
        run = lambda a, b: [reference_block(orc, tiny, wt, ids0, 0, z, z, threads=1) for _ in range(a, b)]
        leg = CpuLeg(run, 1, 4 * (4 * 256 * 256 + 3 * 256 * 688), "block calls of 32 tokens",
                     tokens=32, split=False)
        legs["decoder_c1_seq32"] = legs["decoder_c1_seq32_graph"] = leg
    big_names = ("decoder_c5_prefill512", "decoder_c5_decode_kv2048",
                 "decoder_c5_decode_kv2048_graph", "decoder_c5_decode_kv2048_bf16w")
    if want(*big_names):
        big = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
        wb = {n: (np.ones(sh, np.float32) if n.endswith("norm") else normal(sh, 0.02))
              for n, sh in big.weight_shapes().items()}
        threads = host_threads()
        if want("decoder_c5_prefill512"):
            seq = 64
            ids_p = rng.integers(0, 32000, seq).astype(np.float32)
            zp = np.zeros((seq, 4096), np.float32)
            flops = 2.0 * seq * (4 * 4096 * 4096 + 3 * 4096 * 11008) + 4.0 * 128 * seq * (seq + 1) / 2 * 32
            seq1 = 8  # the single-thread sample: an 8-token prefill
            ids_1 = ids_p[:seq1]
            z1 = np.zeros((seq1, 4096), np.float32)
            flops1 = (2.0 * seq1 * (4 * 4096 * 4096 + 3 * 4096 * 11008)
                      + 4.0 * 128 * seq1 * (seq1 + 1) / 2 * 32)
            legs["decoder_c5_prefill512"] = CpuLeg(
                lambda a, b: [reference_block(orc, big, wb, ids_p, 0, zp, zp, threads=threads)
                              for _ in range(a, b)],
                1, flops, "block calls of a 64-token prefill (the 512-token call's products "
                          "split by rows over threads)", tokens=seq, split=False, cores=threads,
                single=lambda a, b: [reference_block(orc, big, wb, ids_1, 0, z1, z1, threads=1)
                                     for _ in range(a, b)],
                single_what="block calls of an 8-token prefill on one thread",
                single_work=flops1, single_tokens=seq1)
        kc, vc = normal((2049, 4096), 0.5), normal((2049, 4096), 0.5)
        ids_d = rng.integers(0, 32000, 1).astype(np.float32)
        weight_bytes = 4 * (4 * 4096 * 4096 + 3 * 4096 * 11008)
        dec = CpuLeg(lambda a, b: [reference_block(orc, big, wb, ids_d, 2048, kc, vc, threads=1)
                                   for _ in range(a, b)],
                     1, weight_bytes + 2 * 2049 * 4096 * 4, "decode steps at KV 2048", tokens=1,
                     split=False)
        legs["decoder_c5_decode_kv2048"] = legs["decoder_c5_decode_kv2048_graph"] = dec
        legs["decoder_c5_decode_kv2048_bf16w"] = CpuLeg(
            dec.run, 1, weight_bytes // 2 + 2 * 2049 * 4096 * 4,
            "decode steps at KV 2048 (over the widened f32 weights)", tokens=1, split=False)
    return {n: leg for n, leg in legs.items() if n in names}


def _reshape(arr, shape):
    from magnetar_hip.device import DeviceArray
    return DeviceArray(arr.device, arr.ptr, shape, arr.dtype, arr.half, owned=False)


def _fill_normal(dev, arr, s):
    """Fills a large device array chunk by chunk from the seeded generator."""
    from oracle import oracle as orc
    import ctypes
    from magnetar_hip._lib import call
    rows = arr.shape[0]
    chunk = max(1, (64 << 20) // (arr.shape[1] * 4))
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        host = orc.normal((r1 - r0) * arr.shape[1], s + r0)
        call("mhip_upload", dev.ctx, ctypes.c_void_p(arr.ptr + r0 * arr.shape[1] * 4),
             host.ctypes.data_as(ctypes.c_void_p), host.nbytes)


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--only", default="", help="comma-separated kernel names")
    parser.add_argument("--exclude", default="", help="comma-separated kernel names to skip")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    parser.add_argument("--preheat", type=float, default=PREHEAT_S,
                        help="untimed seconds of GPU time each case runs first (clock ramp)")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1"}))
        sys.exit(2)

    import magnetar_hip
    from oracle import oracle as orc

    dev = magnetar_hip.Device(0)
    info = dev.info()
    only = set(filter(None, args.only.split(",")))
    exclude = set(filter(None, args.exclude.split(",")))
    wanted = lambda prefix: not only or any(name.startswith(prefix) for name in only)
    cases = []
    if wanted("matmul"):
        cases += matmul_cases(dev, orc)
    if wanted("attention"):
        cases += attention_cases(dev, orc)
    if not only or only - {c for c in only if c.startswith(("matmul", "attention", "decoder",
                                                             "calibration", "greedy", "kv_write"))}:
        cases += streaming_cases(dev, orc)
    if wanted("greedy") or wanted("kv_write"):
        cases += selection_cases(dev, orc)
    if wanted("decoder"):
        graphs = not {"decoder_c1_seq32_graph", "decoder_c5_decode_kv2048_graph"} <= exclude
        cases += decoder_cases(dev, orc, graphs)
    if any(name.startswith("calibration") for name in only):
        cases += calibration_cases(dev, orc)
    results = {}
    for case in cases:
        if (only and case.name not in only) or case.name in exclude:
            continue
        results[case.name] = case.measure(dev, args.steps, args.warmup, args.preheat)
        r = results[case.name]
        extra = f"  {r['tokens_per_s']:10.1f} tokens/s" if "tokens_per_s" in r else ""
        print(f"# {case.name:14s} {r['ms']*1e3:9.1f} us  {r['achieved']:8.1f} {r['unit']}  "
              f"{100*r['frac']:5.1f}% of {r['bound']}{extra}  host {r['host_us']:.1f} us/call",
              file=sys.stderr, flush=True)
    dev.check_flags()

    head = results.get(HEADLINE)
    roofline = None
    if head:
        roofline = {"bound": "mfma", "achieved": round(head["achieved"], 2),
                    "peak": head["peak"], "unit": head["unit"],
                    "frac": round(head["frac"], 4), "traffic": TRAFFIC.get(HEADLINE)}
    base = None if args.no_cpu or HEADLINE not in results else cpu_baseline(orc)
    if not args.no_cpu:
        threads = _host_threads()
        legs = cpu_legs(orc, set(results))
        for name, leg in legs.items():
            r = results[name]
            r["cpu"] = time_cpu_leg(leg, r["bound"], threads)
            c = r["cpu"]
            print(f"# cpu {name:14s} {c['value']:10.4f} {c['unit']} on {c['cores']} threads"
                  + (f"  {c['tokens_per_s']:.2f} tokens/s" if "tokens_per_s" in c else ""),
                  file=sys.stderr, flush=True)
    line = {
        "metric": METRIC,
        "value": round(head["achieved"], 2) if head else None,
        "unit": head["unit"] if head else None,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "preheat_s_per_case": args.preheat,
        "ms_per_step": round(head["ms"], 5) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: splitmix64/Box-Muller seeded inputs",
        "config": {"workload": "C2 f32 matmul C[4096,4096] = A[4096,4096] B[4096,4096], "
                               "row-major, entries U(-1,1)"},
        "roofline": roofline,
        "cpu_baseline": base,
        "device": {"name": info["name"], "arch": info["architecture"],
                   "compute_units": info["compute_units"]},
        "kernels": {k: dict({"ms": round(v["ms"], 5), "achieved": round(v["achieved"], 2),
                             "unit": v["unit"], "frac": round(v["frac"], 4), "shape": v["shape"],
                             "windows": v["windows"], "host_us": v["host_us"]},
                            **({"tokens_per_s": round(v["tokens_per_s"], 1)}
                               if "tokens_per_s" in v else {}),
                            **({"cpu": v["cpu"]} if "cpu" in v else {}))
                    for k, v in results.items()},
        "cpu_host": {"cpu_model": _cpu_model(), "nproc": os.cpu_count(),
                     "threads": _host_threads()},
    }
    print(json.dumps(line))
    dev.close()


if __name__ == "__main__":
    main()
