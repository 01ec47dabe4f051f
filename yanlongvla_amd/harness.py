"""Stage timing and kernel-class accounting of the deploy path (the reference's runner.capture / timed / kernel_classes,
deploy/tcq_kernels/runner.py:204-266): capture a stage as a HIP graph, time its replays with events, and split the device
time of one replay by kernel class from a profiler trace.

The class patterns name this library's kernels (include/tcq_api.h); anything else falls through to the library classes.
"""
import re
import time
from collections import Counter, defaultdict

import numpy as np
import torch

CLASSES = [
    ('tcq decode', r'k_decode'),
    ('tcq scale+rotate', r'k_post'),
    ('tcq MLP middle', r'k_mid|k_pre2'),
    ('tcq rotate+quantize', r'k_pre|k_norm_pre|k_rht|k_quantize'),
    ('tcq decode+product', r'k_gemm_small<0|k_gemv_tcq|k_gemv_f16'),
    ('tcq product (INT8 weights)', r'k_gemm_small<1'),
    ('int8 matrix product', r'k_gemm_i8'),
    ('bf16 matrix product', r'k_gemm_bf16'),
    ('attention', r'k_attn'),
    ('norm', r'rmsnorm'),
    ('copies / casts', r'copy|cast|Copy|fill|zero|memset|Memset|memcpy|Memcpy|elementwise|vectorized'),
    ('other', r'.*'),
]


def capture(fn, per_graph=1):
    """A HIP graph of per_graph back-to-back calls of fn (one eager call on a side stream first, as capture wants)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    return g


def timed(graph, warmup=20, n=200):
    """Replay statistics in ms: `warmup` untimed replays, then `n` replays each bracketed by events (runner.py:214-224)."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    values = []
    for _ in range(n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        values.append(a.elapsed_time(b))
    v = np.array(values)
    return dict(median_ms=float(np.median(v)), p95_ms=float(np.percentile(v, 95)), mean_ms=float(v.mean()),
                min_ms=float(v.min()), n=n, warmup=warmup)


def warm(fn, seconds, min_calls=1):
    """Call fn until `seconds` of wall time have passed (device synchronised) and at least min_calls calls were made: the
    clocks reach their loaded state before a timed region starts. Returns (calls, seconds)."""
    t0 = time.perf_counter()
    calls = 0
    while True:
        fn()
        calls += 1
        if calls >= min_calls and calls % 8 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= seconds:
                break
    torch.cuda.synchronize()
    return calls, time.perf_counter() - t0


def action_table(actions, reference):
    """Action agreement of every row with the reference row (parity.py:92-99): `actions` maps a row name to an array of
    shape (observations, ...). Per row: observations whose actions are identical, the largest absolute difference, and the
    relative error ||A - A_ref|| / ||A_ref|| per observation (max, mean) and pooled over all observations."""
    ref = np.asarray(actions[reference], dtype=np.float64)
    n = len(ref)
    ref_norm = np.linalg.norm(ref.reshape(n, -1), axis=1)
    table = {}
    for row, a in actions.items():
        a = np.asarray(a, dtype=np.float64)
        if a.shape != ref.shape:
            raise ValueError(f'{row}: actions {a.shape} != reference {ref.shape}')
        d = a - ref
        per = np.linalg.norm(d.reshape(n, -1), axis=1) / ref_norm
        table[row] = dict(identical_observations=int(sum(np.array_equal(x, y) for x, y in zip(a, ref))),
                          max_abs=float(np.abs(d).max()), rel_err_max=float(per.max()), rel_err_mean=float(per.mean()),
                          rel_err_pooled=float(np.linalg.norm(d) / np.linalg.norm(ref)))
    return table


def classify(name):
    return next(c for c, pat in CLASSES if re.search(pat, name))


def kernel_classes(graph=None, fn=None):
    """Device time per kernel class of one replay of `graph` (or one eager call of `fn`), launches, wall time and the
    gaps between kernels, from a torch.profiler trace (ROCm tracer). If a graph replay yields no kernel records, the eager
    call is traced instead (same kernels; launches then include host submission)."""
    from torch.profiler import profile, ProfilerActivity

    def trace(run):
        for _ in range(3):
            run()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with profile(activities=[ProfilerActivity.CUDA, ProfilerActivity.CPU]) as prof:
            a.record()
            run()
            b.record()
            b.synchronize()
        kern = [e for e in prof.events() if e.device_type.name == 'CUDA']
        return a.elapsed_time(b), kern

    mode = 'graph replay'
    wall, kern = trace(graph.replay) if graph is not None else (0.0, [])
    if not kern and fn is not None:
        mode = 'eager call'
        wall, kern = trace(fn)
    by, launches, top = defaultdict(float), Counter(), Counter()
    for e in kern:
        dur = e.time_range.elapsed_us() / 1000
        cls = classify(e.name)
        by[cls] += dur
        launches[cls] += 1
        top[e.name.split('(')[0][:90]] += dur
    total = sum(by.values())
    return dict(traced=mode, wall_ms=round(wall, 4), kernel_ms=round(total, 4), gaps_ms=round(max(wall - total, 0.0), 4),
                launches=sum(launches.values()),
                by_class_ms={k: round(v, 4) for k, v in sorted(by.items(), key=lambda kv: -kv[1])},
                launches_by_class=dict(launches), top=[(n, round(d, 4)) for n, d in top.most_common(8)])
