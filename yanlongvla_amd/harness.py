"""Stage timing and kernel-class accounting of the deploy path. It reports what the reference's harness reports
(deploy/tcq_kernels/runner.py:214-266: 20 + 200 graph replays, median / p95; device time per kernel class of one stage;
parity.py:92-99: action agreement per row), under the same result keys so that figures can be set side by side.

  capture(fn, per_graph)    a HIP graph of per_graph back-to-back calls of fn
  timed(graph)              isolated replays: each starts on an idle device and is bracketed by its own pair of events
  warm(fn, seconds)         calls until the clocks have settled
  kernel_classes(graph, fn) one stage's device time folded from per-kernel totals into classes of this library's kernels
  action_table(actions, r)  agreement of every runtime's actions with runtime r, per observation and pooled
"""
import re
import time

import numpy as np
import torch

# (class, pattern) pairs, first match wins; the patterns name this library's kernels (include/tcq_api.h), then the
# library kernels PyTorch launches between them.
CLASSES = [
    ('tcq decode', r'k_decode'),
    ('tcq scale+rotate', r'k_post'),
    ('tcq MLP middle', r'k_mid|k_pre2'),
    ('tcq rotate+quantize', r'k_pre|k_norm_pre|k_rht|k_quantize'),
    ('tcq decode+product', r'k_gemm_small<0|k_gemv_tcq|k_gemv_f16'),
    ('tcq product (INT8 weights)', r'k_gemm_small<1'),
    ('int8 matrix product', r'k_gemm_i8'),
    ('bf16 matrix product', r'k_gemm_bf16|k_gemm_small<2|k_gemm_small<3'),
    ('attention', r'k_attn'),
    ('norm', r'rmsnorm'),
    ('copies / casts', r'copy|cast|Copy|fill|zero|memset|Memset|memcpy|Memcpy|elementwise|vectorized'),
    ('other', r'.*'),
]
_COMPILED = [(c, re.compile(p)) for c, p in CLASSES]


def classify(name):
    for cls, pat in _COMPILED:
        if pat.search(name):
            return cls
    return 'other'


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


def _quantile(ordered, q):
    """q-quantile of an ascending list, interpolating linearly between the two nearest ranks."""
    pos = q * (len(ordered) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(ordered) - 1)
    return ordered[lo] + (ordered[hi] - ordered[lo]) * (pos - lo)


def timed(graph, warmup=20, n=200):
    """Replay statistics in ms over n isolated replays after `warmup` untimed ones. The event pairs are made before the
    first replay; every timed replay starts on an idle device, so each figure includes the graph's submission."""
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for _ in range(warmup):
        graph.replay()
    for start, end in marks:
        torch.cuda.synchronize()
        start.record()
        graph.replay()
        end.record()
    torch.cuda.synchronize()
    ms = sorted(start.elapsed_time(end) for start, end in marks)
    return dict(median_ms=float(_quantile(ms, 0.5)), p95_ms=float(_quantile(ms, 0.95)), mean_ms=float(sum(ms) / n),
                min_ms=float(ms[0]), n=n, warmup=warmup)


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
    """Agreement of every row's actions with the reference row's. `actions` maps a row name to an array of shape
    (observations, ...). Per row: the observations whose actions are identical, the largest absolute difference, and the
    relative L2 error ||A - A_ref|| / ||A_ref|| per observation (max, mean) and over all observations at once."""
    ref = np.asarray(actions[reference], dtype=np.float64)
    axes = tuple(range(1, ref.ndim))
    ref_sq = np.square(ref).sum(axis=axes)
    table = {}
    for row, a in actions.items():
        a = np.asarray(a, dtype=np.float64)
        if a.shape != ref.shape:
            raise ValueError(f'{row}: actions {a.shape} != reference {ref.shape}')
        d = a - ref
        d_sq = np.square(d).sum(axis=axes)
        rel = np.sqrt(d_sq / ref_sq)
        table[row] = dict(identical_observations=int(np.count_nonzero((a == ref).all(axis=axes))),
                          max_abs=float(np.abs(d).max()), rel_err_max=float(rel.max()), rel_err_mean=float(rel.mean()),
                          rel_err_pooled=float(np.sqrt(d_sq.sum() / ref_sq.sum())))
    return table


def _kernel_totals(run):
    """(wall ms of one traced call of run, [(kernel name, launches, device ms)]) from the profiler's per-name averages."""
    from torch.autograd import DeviceType
    from torch.profiler import ProfilerActivity, profile
    run()
    run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # device activity only: the kernels are all that is read back, and without host activity the tracer links no host
    # launches to device records (that linking warned of duplicate flow starts on ROCm)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        start.record()
        run()
        end.record()
        torch.cuda.synchronize()
    rows = [(k.key, k.count, k.device_time_total / 1e3) for k in prof.key_averages() if k.device_type == DeviceType.CUDA]
    return start.elapsed_time(end), rows


def kernel_classes(graph=None, fn=None):
    """Device time per kernel class of one replay of `graph` (or one eager call of `fn`), with launches, the wall time of
    the traced call and the time between kernels. On ROCm the tracer records no kernels inside graph replays; the eager
    call of the same stage is then traced (same kernels; its wall time includes host submission)."""
    mode, wall, rows = 'graph replay', 0.0, []
    if graph is not None:
        wall, rows = _kernel_totals(graph.replay)
    if not rows and fn is not None:
        mode = 'eager call'
        wall, rows = _kernel_totals(fn)
    classes = {}
    for name, count, ms in rows:
        c = classes.setdefault(classify(name), [0, 0.0])
        c[0] += count
        c[1] += ms
    total = sum(ms for _, ms in classes.values())
    ordered = sorted(classes.items(), key=lambda kv: kv[1][1], reverse=True)
    top = sorted(((name.split('(')[0][:90], ms) for name, _, ms in rows), key=lambda r: r[1], reverse=True)[:8]
    return dict(traced=mode, wall_ms=round(wall, 4), kernel_ms=round(total, 4), gaps_ms=round(max(wall - total, 0.0), 4),
                launches=sum(c for c, _ in classes.values()),
                by_class_ms={k: round(ms, 4) for k, (_, ms) in ordered},
                launches_by_class={k: c for k, (c, _) in ordered}, top=[(n, round(ms, 4)) for n, ms in top])
