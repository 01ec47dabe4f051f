"""Benchmark of the TCQ 2-bit deploy path on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--layers 1024] [--cpu-seconds 10]

Headline workload (one JSON line on stdout): the 2-bit TCQ decode-GEMV of a 2048 x 2048 layer at batch 1 with FP16
activations and the FP16 512 x 2 codebook (bitshift trellis L = 16, K = 2, V = 2), streamed over `--layers` distinct layers
(1 MiB of packed words each; 1024 layers = 1 GiB, four times the 256 MB Infinity Cache, so the words come from HBM). One
step = the complete layer forward of every layer on the same input token:
    input rotation h = fwht(x * su) -> FP16 (tcq_pre_h16, once: the layers share the input signs, as a q/k/v group does)
    fused decode-GEMV and output rotation y_l = fwht((h Q_l^T) * r_l) * sv_l for all layers (tcq_gemv_f16_post, one launch,
    one workgroup per layer).
value = packed-weight bytes per step / step time (GB/s), after at least --warmup steps and --warmup-seconds of warm-up.
roofline = the fused decode-GEMV kernel alone, timed with HIP events on the stream it runs on. cpu_baseline = the oracle's
restatement of the reference layer (reference_linear, FP16 table, unquantized activations) timed on the host over a bounded
sample of the same layers.

Secondary workloads in the same line: the RHT shapes and the W8A8 GEMM (`ops`, each with a CPU baseline of the oracle), the
pi0.5-shaped action-expert chunk (`action_chunk`) and the Gemma-2B-shaped backbone (`backbone`: prefill + 32 decode tokens,
per-product decode rates at one token, a CPU baseline), with the device time by kernel class of each stage
(yanlongvla_amd/harness.py).
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published peak
M_DIM = N_DIM = 2048           # config: one 2048 x 2048 layer, batch 1
PACKED_BYTES = M_DIM * N_DIM * 2 // 8


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=200)
    p.add_argument('--warmup', type=int, default=20)
    p.add_argument('--warmup-seconds', type=float, default=3.0,
                   help='minimum wall time of the headline warm-up (the clocks reach their loaded state first)')
    p.add_argument('--layers', type=int, default=1024)
    p.add_argument('--cpu-seconds', type=float, default=10.0)
    p.add_argument('--no-cpu', action='store_true')
    p.add_argument('--seed', type=int, default=0)
    p.add_argument('--chunk-replays', type=int, default=100)
    p.add_argument('--no-chunk', action='store_true', help='skip the action-expert chunk measurement')
    p.add_argument('--no-ops', action='store_true', help='skip the RHT and W8A8 GEMM measurements')
    p.add_argument('--no-backbone', action='store_true', help='skip the Gemma-2B-shaped backbone measurement')
    p.add_argument('--backbone-replays', type=int, default=10)
    p.add_argument('--probe', choices=('gate_up', 'qkv', 'gate_up_dot4', 'qkv_dot4', 'mid2', 'gemm', 'prefill', 'decode', 'chunk',
                                       'layer'),
                   help='only run one kernel kind --probe-reps times (for rocprofv3 counter passes): the fused decode '
                        'product of one token at the backbone gate/up (32768 x 2048, k_gemv_tcq) or q/k/v (2560 x 2048, '
                        'k_gemm_small) shape over distinct weight sets, the one-token GeGLU middle (16384 wide, '
                        'k_mid2_tw2), the W8A8 GEMM 800 x 2048 x 16384 (k_gemm_i8, int32 out) over distinct weights, or '
                        'the backbone\'s 800-token prefill (fly) or its 32 decode steps as one graph, or one action chunk '
                        '(fly) as one graph, or 100 steps of the single 2048 x 2048 FP16-table layer (two launches each) '
                        'as one graph')
    p.add_argument('--probe-reps', type=int, default=10)
    p.add_argument('--classes', choices=('chunk', 'backbone'), default=None,
                   help='child mode of the bench: print the kernel classes of the fly stages of one workload as JSON')
    p.add_argument('--copy-calibration', action='store_true',
                   help='only run a plain 1 GiB device-to-device copy 8 times (the reference kernel for scaling the '
                        'FETCH_SIZE / WRITE_SIZE counters into bytes)')
    return p.parse_args()


# HBM bytes per launch of the stream's decode-GEMV kernel, from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over
# this benchmark at its default 1024 layers, each scaled by what the counter reads for a plain copy of known size
TRAFFIC_SUMMARY = ROOT / 'profiles' / 'k_gemv_f16_stream1024_traffic.txt'


def traffic_from_profile(nl):
    if nl != 1024 or not TRAFFIC_SUMMARY.exists():
        return None
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if line.startswith('traffic_bytes_per_launch:'):
            return int(line.split(':', 1)[1].strip())
    return None


def copy_calibration():
    import torch
    n = 1 << 30
    src = torch.ones(n, dtype=torch.int8, device='cuda:0')
    dst = torch.empty_like(src)
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_bytes_read': n, 'copy_bytes_written': n, 'copies': 8}), flush=True)


def make_stream(nl, seed, dev):
    """nl synthetic C0 layers: uniform-random packed words, N(0,1) FP16 tables, one FP16 scale per layer drawn U[0.5, 1.5]
    broadcast over rows, random +-1 signs (one shared input sign vector)."""
    import torch
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=dev).manual_seed(seed)
    tiles = (M_DIM // 16) * (N_DIM // 16)
    bits = torch.randint(-32768, 32768, (nl * tiles, 32), generator=g, device=dev, dtype=torch.int32).to(torch.int16)
    wdev = K.repack(bits, nl * M_DIM, N_DIM)                 # stacked layers repack as one tall layer
    per = K.repack_words(M_DIM, N_DIM)
    tlut = torch.randn(nl, 512, 2, generator=g, device=dev).half()
    scale = torch.rand(nl, 1, generator=g, device=dev) + 0.5
    row_scale = scale.expand(nl, M_DIM).half().contiguous()
    su = (torch.randint(0, 2, (N_DIM,), generator=g, device=dev) * 2 - 1).to(torch.int8)
    sv = (torch.randint(0, 2, (nl, M_DIM), generator=g, device=dev) * 2 - 1).to(torch.int8)
    return dict(bits=bits, wdev=wdev, per=per, tlut=tlut, row_scale=row_scale, su=su, sv=sv)


class Stream:
    """Buffers and launch descriptors of one pass over the layer stream (allocated once; the pass allocates nothing)."""

    def __init__(self, L, x, M=1, fused=True):
        import torch
        from yanlongvla_amd import kernels as K
        dev = x.device
        nl = L['tlut'].shape[0]
        self.K, self.L, self.x, self.nl, self.M = K, L, x, nl, M
        self.h16 = torch.empty(M, N_DIM, dtype=torch.float16, device=dev)
        self.hs = torch.empty(M, dtype=torch.float32, device=dev)
        self.z = torch.empty(nl, M, M_DIM, dtype=torch.float32, device=dev)
        self.y = torch.empty(nl, M, M_DIM, dtype=torch.float16, device=dev)
        w = L['wdev'].view(nl, L['per'])
        self.fused = fused
        self.gdesc = K.gemv_descriptors([(w[i], L['tlut'][i], L['row_scale'][i], self.z[i]) for i in range(nl)])
        self.pdesc = K.post_segments([(self.z[i], 0, None, L['sv'][i], None, self.y[i], False) for i in range(nl)], dev)
        self.fdesc = K.gemv_post_descriptors([(w[i], L['tlut'][i], L['row_scale'][i], L['sv'][i], None, self.y[i])
                                              for i in range(nl)])

    def rotate_in(self):
        self.K.pre_h16(self.x, self.L['su'], self.h16, self.hs)

    def gemv(self):
        if self.fused:
            import torch
            self.K.gemv_f16_post(self.fdesc, self.h16, self.hs, M_DIM, N_DIM, torch.float16)
        else:
            self.K.gemv_f16(self.gdesc, self.h16, self.hs, M_DIM, N_DIM)

    def rotate_out(self):
        import torch
        self.K.post_batched(self.pdesc, self.nl, torch.float32, torch.float16, None, self.M, M_DIM)

    def step(self):
        self.rotate_in()
        self.gemv()
        if not self.fused:
            self.rotate_out()


def timed(fn, steps, warmup, warm_seconds=0.0):
    """Average ms of fn over `steps` calls after at least `warmup` untimed calls and `warm_seconds` of warm-up wall time,
    HIP events on the current stream (where the library launches), bracketed by device synchronisation."""
    import torch
    from yanlongvla_amd import harness
    harness.warm(fn, warm_seconds, warmup)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def capture(fn, per_graph=1):
    """A HIP graph of per_graph back-to-back calls of fn (one eager call on a side stream first, as graph capture wants)."""
    import torch
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


def graph_latency(fn, replays=200, warmup=20, per_graph=1):
    """Median / p95 ms per call of fn from HIP-graph replays (the reference's timing protocol: 20 warm-up + 200 timed
    replays, each bracketed by events, so each includes the graph's submission). With per_graph > 1 the graph holds that
    many calls back to back and the replay time is divided by it."""
    import torch
    g = capture(fn, per_graph)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) / per_graph)
    ts.sort()
    return ts[len(ts) // 2], ts[int(len(ts) * 0.95)]


def check_against_oracle(L, S, n_check=2):
    """Spot check of the timed pass: the first layers' outputs against the oracle (relative L2 <= 2e-3)."""
    import numpy as np
    from oracle import tcq_oracle as O
    x = S.x.float().cpu().numpy()
    errs = []
    for i in range(n_check):
        OL = oracle_layer(L, i)
        ref = O.reference_linear(x, OL, a8=False, table='fp16', out_dtype='f32')
        y = S.y[i].float().cpu().numpy()
        errs.append(float(np.linalg.norm(y - ref) / np.linalg.norm(ref)))
    return max(errs)


def oracle_layer(L, i):
    from oracle import tcq_oracle as O
    tiles = (M_DIM // 16) * (N_DIM // 16)
    t = dict(bits=L['bits'][i * tiles:(i + 1) * tiles].cpu().numpy(), tlut=L['tlut'][i].cpu().numpy(),
             row_scale=L['row_scale'][i].cpu().numpy(), su=L['su'].cpu().numpy(), sv=L['sv'][i].cpu().numpy())
    return O.Layer(f'layer{i}', t)


def cpu_baseline(L, x, seconds):
    """The oracle's reference layer (FP16 table, a8=False: windowed read, table lookup, FP64 product, two rotations) on the
    host cores, over as many of the stream's layers as fit in about `seconds` (at least 2)."""
    import numpy as np
    from oracle import tcq_oracle as O
    try:
        from threadpoolctl import threadpool_info
        blas = max([d.get('num_threads', 1) for d in threadpool_info() if d.get('user_api') == 'blas'] or [1])
    except Exception:
        blas = 1
    xs = x.float().cpu().numpy()
    layers = [oracle_layer(L, 0)]
    O.reference_linear(xs, layers[0], a8=False, table='fp16', out_dtype='f32')      # warm-up
    el, done = 0.0, 0          # compute time only: the device -> host copy of each layer is outside the timing
    while done < 2 or (el < seconds and done < L['tlut'].shape[0]):
        OL = oracle_layer(L, done)
        t1 = time.perf_counter()
        O.reference_linear(xs, OL, a8=False, table='fp16', out_dtype='f32')
        el += time.perf_counter() - t1
        done += 1
    return dict(value=round(done * PACKED_BYTES / el / 1e9, 4), unit='GB/s', cores=int(blas), kind='port',
                sample=f'{done} of the stream\'s 2048x2048 layers at batch 1 through the numpy oracle '
                       f'(reference_linear, FP16 table, a8=False), {el:.1f} s; host affinity {len(os.sched_getaffinity(0))} cores')


# ------------------------------------------------------------------------------------------------ RHT and W8A8 GEMM
MFMA_I8_PEAK_TOPS = 5000.0     # MI355X dense INT8 MFMA, published peak


def graph_per_call(fn, calls=20, replays=20):
    """Device ms per call of fn: a HIP graph of `calls` back-to-back calls replayed `replays` times back to back between two
    events. One untimed replay runs first, so the GPU is busy while the host queues the timed ones and no submission gap
    falls inside the timed region; the total is divided by replays x calls."""
    import torch
    g = capture(fn, calls)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g.replay()
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / (replays * calls)


ROTATE_BYTES = 512 << 20        # distinct operands per timed graph: twice the 256 MB last-level cache
ROTATE_MAX_SETS = 512


def rotating_sets(bytes_per_set):
    """How many distinct operand sets of this size one timed graph cycles through: enough for ROTATE_BYTES (each call
    then finds its operands outside the last-level cache), at most ROTATE_MAX_SETS."""
    return max(2, min(ROTATE_MAX_SETS, -(-ROTATE_BYTES // bytes_per_set)))


def rotating_per_call(fns, replays=5):
    """Device ms per call of a list of calls on distinct operands, captured in order as one graph (graph_per_call)."""
    def run():
        for f in fns:
            f()
    return graph_per_call(run, calls=1, replays=replays) / len(fns)


def hbm_figure(byts, ms, sets):
    """The rate of a call over distinct operands: an HBM fraction when the sets exceed the last-level cache."""
    gbs = byts / (ms * 1e-3) / 1e9
    r = {'us': round(ms * 1e3, 2), 'GBs': round(gbs, 1), 'distinct_operand_MB': round(sets * byts / 2 ** 20, 1), 'sets': sets}
    if sets * byts > 256 << 20:
        r['hbm_frac'] = round(gbs / HBM_PEAK_GBS, 4)
    else:
        r['note'] = 'operands fit the last-level cache even across sets: launch / latency bound, no HBM figure'
    return r


def rht_figures(dev, seed):
    """Randomized block-Walsh transform of BF16 rows [M, n] (tcq_rht, BF16 in and out), per call; bytes = 4 M n + n. Timed
    over distinct input / output rows (rotating_sets) and, labelled cache-resident, on one set."""
    import torch
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=dev).manual_seed(seed + 5)
    out = {}
    for n in (1024, 2048, 4096, 16384):
        su = (torch.randint(0, 2, (n,), generator=g, device=dev) * 2 - 1).to(torch.int8)
        for M in (1, 16, 50, 800):
            byts = 4 * M * n + n
            S = rotating_sets(byts)
            xs = torch.randn(S, M, n, generator=g, device=dev).bfloat16()
            ys = torch.empty_like(xs)
            ms = rotating_per_call([lambda i=i: K.rht(xs[i], su, ys[i]) for i in range(S)])
            r = hbm_figure(byts, ms, S)
            r['us_cache_resident'] = round(graph_per_call(lambda: K.rht(xs[0], su, ys[0])) * 1e3, 2)
            out[f'{M}x{n}'] = r
            del xs, ys
    torch.cuda.empty_cache()
    return out


def gemm_figures(dev, seed):
    """W8A8 GEMM, K = 2048, N = 16384: A = per-token INT8 of N(0,1) BF16 activations, B = per-channel INT8 of N(0, 0.02)
    weights (tcq_quantize_rows); timed: the exact int32 product and the BF16 output (acc * s_token) * s_channel, over
    distinct weight / activation sets (rotating_sets; the same-operand times are reported as cache-resident). The
    M = 50 product is checked bit-exact against the oracle's integer matmul."""
    import numpy as np
    import torch
    from oracle import tcq_oracle as O
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=dev).manual_seed(seed + 6)
    Kd, N = 2048, 16384
    wbytes = N * Kd + 4 * N
    SW = rotating_sets(wbytes)
    qw = torch.empty(SW, N, Kd, dtype=torch.int8, device=dev)
    sw = torch.empty(SW, N, dtype=torch.float32, device=dev)
    for i in range(SW):
        w = (torch.randn(N, Kd, generator=g, device=dev) * 0.02).bfloat16()
        K.quantize_rows(w, qw[i], sw[i])
    del w
    out = {}
    for M in (800, 50, 1):
        a = torch.randn(SW, M, Kd, generator=g, device=dev).bfloat16()
        qa = torch.empty(SW, M, Kd, dtype=torch.int8, device=dev)
        sa = torch.empty(SW, M, dtype=torch.float32, device=dev)
        for i in range(SW):
            K.quantize_rows(a[i], qa[i], sa[i])
        acc = torch.empty(M, N, dtype=torch.int32, device=dev)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        t_i32 = rotating_per_call([lambda i=i: K.gemm_i8(qa[i], qw[i], acc) for i in range(SW)])
        t_bf16 = rotating_per_call([lambda i=i: K.gemm_i8(qa[i], qw[i], y, sa[i], sw[i]) for i in range(SW)])
        c_i32 = graph_per_call(lambda: K.gemm_i8(qa[0], qw[0], acc))
        c_bf16 = graph_per_call(lambda: K.gemm_i8(qa[0], qw[0], y, sa[0], sw[0]))
        ops = 2 * M * N * Kd
        byts = M * Kd + N * Kd + 4 * M + 4 * N + 2 * M * N
        r = {'us_int32': round(t_i32 * 1e3, 2), 'us_bf16': round(t_bf16 * 1e3, 2),
             'TOPS_bf16': round(ops / (t_bf16 * 1e-3) / 1e12, 1), 'GBs_bf16': round(byts / (t_bf16 * 1e-3) / 1e9, 1),
             'distinct_weight_sets': SW, 'distinct_operand_MB': round(SW * (byts - 2 * M * N) / 2 ** 20, 1),
             'us_int32_cache_resident': round(c_i32 * 1e3, 2), 'us_bf16_cache_resident': round(c_bf16 * 1e3, 2)}
        if M == 800:
            r['mfma_frac_bf16'] = round(r['TOPS_bf16'] / MFMA_I8_PEAK_TOPS, 4)
            r['mfma_frac_int32'] = round(ops / (t_i32 * 1e-3) / 1e12 / MFMA_I8_PEAK_TOPS, 4)
            # the reference's own prefill product (torch._int_mm, hipBLASLt on ROCm) on the same operand sets and box
            try:
                K.gemm_i8(qa[0], qw[0], acc)
                same = bool(torch.equal(torch._int_mm(qa[0], qw[0].t()), acc))
                r['torch_int_mm_us_int32'] = round(rotating_per_call([lambda i=i: torch._int_mm(qa[i], qw[i].t())
                                                                      for i in range(SW)]) * 1e3, 2)
                r['torch_int_mm_equal'] = same
            except RuntimeError as e:
                r['torch_int_mm_us_int32'] = f'unavailable: {e}'[:120]
        else:
            r['hbm_frac_bf16'] = round(r['GBs_bf16'] / HBM_PEAK_GBS, 4)
            r['hbm_frac_int32'] = round((byts - 2 * M * N + 4 * M * N) / (t_i32 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        if M == 50:
            K.gemm_i8(qa[0], qw[0], acc)
            K.gemm_i8(qa[0], qw[0], y, sa[0], sw[0])
            ref = O.int_matmul(qa[0].cpu().numpy(), qw[0].cpu().numpy())
            r['int32_bitexact'] = bool(np.array_equal(acc.cpu().numpy(), ref))
            yb = O.bf16_bits((ref.astype(np.float32) * sa[0].cpu().numpy()[:, None]) * sw[0].cpu().numpy()[None, :])
            r['bf16_bitexact'] = bool(np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), yb))
        out[f'M={M}'] = r
        del a, qa, sa
    del qw, sw
    torch.cuda.empty_cache()
    return out


def blas_threads():
    try:
        from threadpoolctl import threadpool_info
        return max([d.get('num_threads', 1) for d in threadpool_info() if d.get('user_api') == 'blas'] or [1])
    except Exception:
        return 1


def rht_cpu_baseline(seed, seconds):
    """The oracle's fwht (tcq_format.py:44-55 restated in numpy) of x * su over BF16 rows [800, 16384] (the largest
    RHT shape), FP32 butterflies and BF16 output, as many repeats as fit in about `seconds` (at least 3, median). The rows
    are split into one slice per host core, each transformed by its own thread (numpy's element-wise loops release the
    interpreter lock), so every core of the box works."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle import tcq_oracle as O
    rng = np.random.default_rng(seed + 5)
    M, n = 800, 16384
    x = O.bf16_to_f32(O.bf16_bits(rng.standard_normal((M, n)).astype(np.float32)))
    su = np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.float32)
    cores = max(1, len(os.sched_getaffinity(0)))
    bounds = np.linspace(0, M, cores + 1).astype(int)
    slices = [(int(a), int(b)) for a, b in zip(bounds[:-1], bounds[1:]) if b > a]
    ts, t0 = [], time.perf_counter()
    with ThreadPoolExecutor(max_workers=len(slices)) as ex:
        while len(ts) < 3 or (time.perf_counter() - t0 < seconds and len(ts) < 20):
            t1 = time.perf_counter()
            list(ex.map(lambda ab: O.bf16_bits(O.fwht(x[ab[0]:ab[1]] * su)), slices))
            ts.append(time.perf_counter() - t1)
    med = float(np.median(ts))
    byts = 4 * M * n + n
    return dict(value=round(byts / med / 1e9, 4), unit='GB/s', cores=len(slices), kind='port',
                sample=f'{len(ts)} transforms of BF16 [{M}, {n}] through the numpy oracle (fwht of x * su, BF16 out), median '
                       f'{med * 1e3:.1f} ms; rows split over {len(slices)} threads, one per host core')


def gemm_cpu_baseline(seed, seconds):
    """The reference's CPU path of the W8A8 product (tcq_format.py:110-122, 135): quantize_tokens of the activations,
    int_matmul's CPU branch (FP64 matmul -> int32), then (acc * s) * s_channel -> BF16, at K = 2048, N = 16384 on as many
    of the 800 token rows as fit in about `seconds` (per-channel weight quantization is offline and not timed)."""
    import numpy as np
    from oracle import tcq_oracle as O
    rng = np.random.default_rng(seed + 6)
    Kd, N = 2048, 16384
    qw, sw = O.quantize_channels((rng.standard_normal((N, Kd)) * 0.02).astype(np.float32))

    def run(M):
        a = O.bf16_to_f32(O.bf16_bits(rng.standard_normal((M, Kd)).astype(np.float32)))
        t1 = time.perf_counter()
        q, s_ = O.quantize_tokens(a)
        acc = O.int_matmul(q, qw)
        O.bf16_bits((acc.astype(np.float32) * s_) * sw[None, :])
        return time.perf_counter() - t1
    t50 = run(50)
    M = int(min(800, max(50, 50 * seconds / 2 / max(t50, 1e-3))))
    el = run(M)
    ops = 2 * M * N * Kd
    return dict(value=round(ops / el / 1e12, 5), unit='TOPS', cores=int(blas_threads()), kind='port',
                sample=f'{M} of the 800 token rows x K {Kd} x N {N} through the numpy oracle (quantize_tokens, FP64 int_matmul, '
                       f'scales, BF16 out), {el:.2f} s; BLAS threads as cores')


# ------------------------------------------------------------------------------------------------ action-expert chunk
CHUNK_TOKENS, CHUNK_STEPS, PREFIX = 50, 10, 800
EXPERT_PACKED_BYTES = 311_427_072 * 2 // 8      # 2-bit payload of the expert's 126 layers, per flow step


def expert_setup(seed, dev):
    """Prefix KV cache (800 rows of keys / values per layer, N(0,1) BF16) and the chunk's noise, seeded."""
    import torch
    from yanlongvla_amd import gemma
    g = torch.Generator(device=dev).manual_seed(seed + 3)
    nl = gemma.EXPERT['layers']
    ks = [torch.randn(PREFIX, 256, generator=g, device=dev).bfloat16() for _ in range(nl)]
    vs = [torch.randn(PREFIX, 256, generator=g, device=dev).bfloat16() for _ in range(nl)]
    noise = torch.randn(CHUNK_TOKENS, gemma.EXPERT['action_dim'], generator=g, device=dev)
    return ks, vs, noise


def expert_policy(runtime, seed, dev, ks, vs):
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.ExpertPolicy, dev, seed=seed)
    model.set_prefix(ks, vs)
    layers = gemma.synthetic_layers(model, seed + 7, dev)        # the same weights for every runtime
    modules.install(model, runtime=runtime, layers=layers)
    return model, layers


def action_chunk(args, dev):
    """ms per action chunk of the 2-bit pi0.5-shaped expert: 18 layers, 50 action tokens against an 800-row prefix KV cache,
    10 Euler steps, captured as one HIP graph per operating point; the fused runtimes are checked bit-exact against the
    layer-by-layer reference runtime on the same chunk."""
    import torch
    from yanlongvla_amd import modules
    ks, vs, noise = expert_setup(args.seed, dev)
    out, res, keep = {}, {}, {}
    with torch.inference_mode():
        for runtime in ('reference', 'fly', 'resident', 'hybrid'):
            model, layers = expert_policy(runtime, args.seed, dev, ks, vs)

            def chunk(model=model, runtime=runtime):
                if runtime == 'hybrid':
                    modules.decode_chunk(model)
                return model.sample_chunk(noise, CHUNK_STEPS)
            out[runtime] = chunk().clone()
            if runtime != 'reference':
                med, p95 = graph_latency(chunk, replays=args.chunk_replays, warmup=10)
                res[runtime] = {'median': round(med, 4), 'p95': round(p95, 4)}
            if runtime == 'fly':
                keep = dict(model=model, layers=layers, classes=traced_classes('chunk', args.seed))
            else:
                del model, layers
            torch.cuda.synchronize()
    exact = {r: bool(torch.equal(out[r], out['reference'])) for r in ('fly', 'resident', 'hybrid')}
    fly = res['fly']['median']
    return dict(workload=f'pi0.5-shaped action expert, 18 layers x (q 2048x1024, k/v 256x1024, o 1024x2048, gate/up '
                         f'4096x1024, down 1024x4096) 2-bit TCQ, {CHUNK_TOKENS} action tokens, {PREFIX}-row prefix KV, '
                         f'{CHUNK_STEPS} Euler steps, one HIP graph per chunk',
                ms_per_chunk=fly, ms_per_chunk_p95=res['fly']['p95'], runtime='fly (2-bit stream decoded on every call)',
                operating_points_ms=res, bitexact_vs_reference_runtime=exact, kernel_classes_fly=keep['classes'],
                packed_bytes_per_chunk=EXPERT_PACKED_BYTES * CHUNK_STEPS,
                effective_packed_GBs=round(EXPERT_PACKED_BYTES * CHUNK_STEPS / (fly * 1e-3) / 1e9, 2)), keep, (ks, vs, noise)


def oracle_linear_class():
    """nn.Module running one quantized Linear through the oracle's reference_linear on the host (W2A8, its INT8 weight
    decoded once at construction, untimed), as RefLinear(resident=True) runs it."""
    import numpy as np
    import torch
    from oracle import tcq_oracle as O

    class OracleLinear(torch.nn.Module):
        def __init__(self, L):
            super().__init__()
            self.ol = O.Layer(L.name, dict(bits=L.bits.cpu().numpy(), tlut=L.tlut.cpu().numpy(),
                                           row_scale=L.row_scale.cpu().numpy(), su=L.su.cpu().numpy(), sv=L.sv.cpu().numpy()))
            self.w8 = L.w8_reference().cpu().numpy()

        def forward(self, x):
            y = O.reference_linear(x.float().reshape(-1, self.ol.n).numpy(), self.ol, w8=self.w8)
            return torch.from_numpy(y.view(np.int16)).view(torch.bfloat16).reshape(*x.shape[:-1], self.ol.m)
    return OracleLinear


def chunk_cpu_baseline(keep, setup, seconds):
    """One flow step of the same expert on the host: every quantized Linear through the oracle's reference_linear with its
    INT8 weight decoded once beforehand (as RefLinear(resident=True)); norms, attention and residuals by PyTorch on the
    CPU. ms per chunk = 10 x the step."""
    import numpy as np
    import torch
    from oracle import tcq_oracle as O
    from yanlongvla_amd import gemma, modules
    model, layers = keep['model'], keep['layers']
    ks, vs, noise = setup

    OracleLinear = oracle_linear_class()
    cpu = gemma.ExpertPolicy().bfloat16().requires_grad_(False)
    state = {k: v.cpu() for k, v in model.state_dict().items()}
    cpu.load_state_dict(state, strict=False)
    cpu.set_prefix([k.cpu() for k in ks], [v.cpu() for v in vs])
    for n, L in layers.items():
        modules.set_submodule(cpu, n, OracleLinear(L))
    x = noise.cpu()
    with torch.inference_mode():
        t0 = time.perf_counter()
        cpu.velocity(x)
        el = time.perf_counter() - t0
    return dict(value=round(el * CHUNK_STEPS * 1e3, 1), unit='ms per chunk', cores=torch.get_num_threads(), kind='port',
                sample=f'one of the chunk\'s {CHUNK_STEPS} flow steps ({el:.1f} s), times {CHUNK_STEPS}: 126 layers through the '
                       f'numpy oracle (reference_linear, INT8 weights decoded once), PyTorch CPU for norms and attention; '
                       f'host affinity {len(os.sched_getaffinity(0))} cores')


# ------------------------------------------------------------------------------------------------------ backbone
BB_IMAGE, BB_TEXT, BB_DECODE = 256, 544, 32
BACKBONE_WEIGHTS = 1_981_808_640


def backbone_setup(seed, dev):
    import torch
    from yanlongvla_amd import gemma
    g = torch.Generator(device=dev).manual_seed(seed + 8)
    img = torch.randn(BB_IMAGE, gemma.BACKBONE['width'], generator=g, device=dev).bfloat16()
    ids = torch.randint(0, gemma.BACKBONE['vocab'], (BB_TEXT,), generator=g, device=dev)
    dec = torch.randint(0, gemma.BACKBONE['vocab'], (BB_DECODE, 1), generator=g, device=dev)
    return img, ids, dec


def backbone(args, dev):
    """Gemma-2B-shaped language model (18 layers, width 2048, MLP 16384, 8 query heads / 1 KV head of dim 256): prefill over
    256 image embeddings + 544 token embeddings, then 32 single-token decode steps on the grown KV cache (synthetic token
    ids). fly = 2-bit TCQ decoded on every call; resident = the W8A8 variant (INT8 weights decoded once at load). Prefill
    and the 32 decode steps are two HIP graphs; fly and resident are checked bit-exact against the reference runtime."""
    import torch
    from yanlongvla_amd import gemma, modules
    img, ids, dec = backbone_setup(args.seed, dev)
    res, outs, products, classes, cpu = {}, {}, {}, {}, None
    with torch.inference_mode():
        for runtime in ('reference', 'fly', 'resident'):
            model = gemma.make_policy(gemma.BackbonePolicy, dev, seed=args.seed + 1)
            layers = gemma.synthetic_layers(model, args.seed + 9, dev)
            modules.install(model, runtime=runtime, layers=layers)
            if runtime != 'fly':
                del layers
            x = torch.cat([img, model.embed(ids)], 0)
            state = {}

            def prefill(model=model, x=x, state=state):
                h, ks, vs = model.prefill(x)
                state.update(h=h, ks=ks, vs=vs)
                return h

            p0 = prefill().clone()
            cache = gemma.KVCache(state['ks'], state['vs'], BB_DECODE)   # the prefill's rows plus room for the decode

            def decode(model=model, cache=cache):
                cache.rewind()
                hs = [model.decode_step_cached(model.embed(dec[t]), cache) for t in range(BB_DECODE)]
                return torch.cat(hs, 0)
            outs[runtime] = (p0, decode().clone())
            if runtime != 'reference':
                p_med, p_p95 = graph_latency(prefill, replays=args.backbone_replays, warmup=2)
                prefill()
                d_med, d_p95 = graph_latency(decode, replays=args.backbone_replays, warmup=2)
                res[runtime] = {'prefill_ms': round(p_med, 3), 'decode_ms_32_tokens': round(d_med, 3),
                                'total_ms': round(p_med + d_med, 3), 'decode_ms_per_token': round(d_med / BB_DECODE, 4)}
                products[runtime] = decode_products(model, runtime, dev, args.seed)
            if runtime == 'fly':
                classes = traced_classes('backbone', args.seed)
                if not args.no_cpu:
                    prefill()
                    cpu = backbone_cpu_baseline(model, layers, x, state, [model.embed(dec[t]) for t in range(2)])
            del model, state
            torch.cuda.synchronize()
    exact = {r: bool(torch.equal(outs[r][0], outs['reference'][0]) and torch.equal(outs[r][1], outs['reference'][1]))
             for r in ('fly', 'resident')}
    tok_fly = res['fly']['decode_ms_per_token']
    return dict(workload='Gemma-2B-shaped backbone, 18 layers x (q 2048x2048, k/v 256x2048, o 2048x2048, gate/up 16384x2048, '
                         'down 2048x16384), 800-token prefill (256 image embeddings + 544 token ids), 32 decode steps',
                runtimes=res, bitexact_vs_reference_runtime=exact,
                prefill_int8_TOPS={r: round(2 * 800 * BACKBONE_WEIGHTS / (v['prefill_ms'] * 1e-3) / 1e12, 1) for r, v in res.items()},
                decode_packed_bytes_per_token=BACKBONE_WEIGHTS // 4,
                decode_effective_packed_GBs_fly=round(BACKBONE_WEIGHTS / 4 / (tok_fly * 1e-3) / 1e9, 1),
                decode_effective_int8_GBs_resident=round(BACKBONE_WEIGHTS / (res['resident']['decode_ms_per_token'] * 1e-3) / 1e9, 1),
                decode_products_M1=products, kernel_classes_fly=classes, cpu_baseline=cpu)


class _Calls(list):
    """A list of calls that also keeps their tensors alive."""
    keep = None


def product_sets(widths, Kd, resident, parts, dev, g, dot=None):
    """Calls of one small-M product shape (segments of the given widths side by side, K = Kd, one token in the token-block
    layout) over distinct synthetic weight sets (rotating_sets): repacked 2-bit words (fly) or INT8 weights (resident),
    each set its own tables and row scales; dot: the product's arithmetic (SmallProduct). Returns (calls, bytes per call,
    sets)."""
    import torch
    from yanlongvla_amd import kernels as K
    Ntot = sum(widths)
    byts = Ntot * Kd if resident else Ntot * Kd // 4
    S = rotating_sets(byts)
    col0 = [sum(widths[:i]) for i in range(len(widths))]
    if parts > 1:
        out = torch.empty(parts, 1, Ntot, dtype=torch.int32, device=dev)
        outs = [out[0, :, c:] for c in col0]
    else:
        out = torch.empty(1, Ntot, dtype=torch.float32, device=dev)
        outs = [out[:, c:] for c in col0]
    x = torch.randn(1, Kd, generator=g, device=dev).bfloat16()
    su = (torch.randint(0, 2, (Kd,), generator=g, device=dev) * 2 - 1).to(torch.int8)
    q4, sc = K.token_blocks(1, Kd, dev), torch.empty(1, dtype=torch.float32, device=dev)
    K.pre(x, su, q4=q4, scale=sc)
    calls, keep = _Calls(), [out, q4, sc]
    for _ in range(S):
        segs = []
        for m, o in zip(widths, outs):
            rs = torch.rand(m, generator=g, device=dev) * 1e-3
            if resident:
                w, t8 = torch.randint(-127, 128, (m, Kd), generator=g, device=dev, dtype=torch.int8), None
            else:
                w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K.repack_words(m, Kd),), generator=g, device=dev, dtype=torch.int32)
                t8 = torch.randint(-127, 128, (512, 2), generator=g, device=dev, dtype=torch.int8)
            segs.append((w, t8, rs, o))
        prod = K.SmallProduct(segs, Ntot, resident=resident)
        calls.append(lambda prod=prod: prod(q4, sc, parts, dot))
        keep.append(prod)
    calls.keep = keep
    return calls, byts, S


def decode_products(model, runtime, dev, seed):
    """Device time and weight-stream rate of each product of the decode step at one token (q/k/v, o, gate/up, down of a
    decoder layer), per call: over distinct weight sets of the layer's shapes (product_sets, more than 256 MB in all, so
    every call streams its weights from HBM; fly reads the 2-bit words, m * n / 4 bytes, resident the INT8 weights), and,
    labelled cache-resident, on decoder layer 0's own group replayed in place. The o and down products run in the K parts
    the decoder layer uses for them (Group.k_parts; their epilogue adds the parts)."""
    import torch
    groups = {g.layers[0].name: g for g in model._tcq_groups}
    pre = 'paligemma_with_expert.paligemma.language_model.layers.0.'
    g0 = torch.Generator(device=dev).manual_seed(seed + 11)
    out = {}
    for tag, key in (('q/k/v', 'self_attn.q_proj'), ('o', 'self_attn.o_proj'), ('gate/up', 'mlp.gate_proj'), ('down', 'mlp.down_proj')):
        g = groups[pre + key]
        resident = runtime != 'fly'
        b = g.quantize(torch.randn(1, g.K, generator=g0, device=dev).bfloat16())
        parts = g.k_parts(1) if tag in ('o', 'down') else 1
        ms_cache = graph_per_call(lambda: g.product(b, parts))
        calls, byts, S = product_sets(g.N, g.K, resident, parts, dev, g0)
        r = hbm_figure(byts, rotating_per_call(calls), S)
        r.update(shape=f'{g.Ntot}x{g.K}', bytes=byts, k_parts=parts, us_cache_resident=round(ms_cache * 1e3, 2))
        out[tag] = r
        del calls
        torch.cuda.empty_cache()
    return out


def backbone_cpu_baseline(model, layers, x, state, dec_x):
    """The backbone on the host, every quantized Linear through the oracle's reference_linear (INT8 weights decoded once,
    untimed), norms and attention by PyTorch on the CPU: decoder layer 0 over the 800-row prefill (times 18) and one decode
    token through all 18 layers against the prefill's KV rows (times 32)."""
    import torch
    from yanlongvla_amd import gemma, modules
    OracleLinear = oracle_linear_class()
    with torch.device('meta'):
        cpu = gemma.BackbonePolicy()
    cpu.embed_tokens = torch.nn.Identity()
    for n, L in layers.items():
        modules.set_submodule(cpu, n, OracleLinear(L))
    cpu = cpu.to_empty(device='cpu').bfloat16().requires_grad_(False)
    for n, p in model.named_parameters():
        if n.endswith('layernorm.weight') or n == 'paligemma_with_expert.paligemma.language_model.norm.weight':
            cpu.get_parameter(n).copy_(p.cpu())
    nl = len(cpu.stack.layers)
    with torch.inference_mode():
        xc = x.cpu()
        t0 = time.perf_counter()
        cpu.stack.layers[0](xc, causal_offset=0)
        t_pre = time.perf_counter() - t0
        ks, vs = [k.cpu() for k in state['ks']], [v.cpu() for v in state['vs']]
        t0 = time.perf_counter()
        cpu.decode_step(dec_x[0].cpu(), ks, vs)
        t_tok = time.perf_counter() - t0
    total = (t_pre * nl + t_tok * BB_DECODE) * 1e3
    return dict(value=round(total, 1), unit='ms (800-token prefill + 32 decode tokens)', cores=torch.get_num_threads(),
                kind='port', prefill_layer_s=round(t_pre, 3), decode_token_s=round(t_tok, 3),
                sample=f'decoder layer 0 of the 800-token prefill ({t_pre:.2f} s, times {nl}) and one decode token through all '
                       f'{nl} layers ({t_tok:.2f} s, times {BB_DECODE}): every quantized Linear through the numpy oracle '
                       f'(reference_linear, INT8 weights decoded once), PyTorch CPU for norms and attention; host affinity '
                       f'{len(os.sched_getaffinity(0))} cores')


def probe(kind, reps, dev):
    """Run one kernel kind `reps` times (see --probe); prints what ran, nothing else."""
    import torch
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=dev).manual_seed(1)
    if kind in ('gate_up', 'qkv', 'gate_up_dot4', 'qkv_dot4'):
        calls, _, _ = product_sets([16384, 16384] if kind.startswith('gate_up') else [2048, 256, 256], 2048, False, 1, dev, g,
                                   dot=kind.endswith('dot4'))
    elif kind == 'mid2':
        N = 16384
        acc = torch.randn(1, 2 * N, generator=g, device=dev) * 0.01
        sv = (torch.randint(0, 2, (2 * N,), generator=g, device=dev) * 2 - 1).to(torch.int8)
        su = (torch.randint(0, 2, (N,), generator=g, device=dev) * 2 - 1).to(torch.int8)
        q4, sc, lut = K.token_blocks(1, N, dev), torch.empty(1, device=dev), K.gelu_table(dev)
        calls = [lambda: K.mid2(acc, None, None, sv, su, q4=q4, scale=sc, gelu_lut=lut)] * 64
    elif kind == 'layer':
        from yanlongvla_amd import harness
        L = make_stream(1, 0, dev)
        x = torch.randn(1, N_DIM, generator=g, device=dev).half()
        S1 = Stream(L, x, fused=False)

        def steps():                              # the two-launch layer: rotation + decode-GEMV, output rotation
            for _ in range(100):
                K.pre_gemv_f16(x, L['su'], L['wdev'], L['tlut'][0], L['row_scale'][0], S1.z[0])
                K.post(S1.z[0], None, None, L['sv'][0], None, S1.y[0])
        g = harness.capture(steps)
        calls = [g.replay]
    elif kind == 'chunk':
        from yanlongvla_amd import harness
        with torch.inference_mode():
            ks, vs, noise = expert_setup(0, dev)
            model, _ = expert_policy('fly', 0, dev, ks, vs)
            g = harness.capture(lambda: model.sample_chunk(noise, CHUNK_STEPS))
        calls = [g.replay]
    elif kind in ('prefill', 'decode'):
        from yanlongvla_amd import gemma, harness, modules
        img, ids, dec = backbone_setup(0, dev)
        with torch.inference_mode():
            model = gemma.make_policy(gemma.BackbonePolicy, dev, seed=1)
            modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, 9, dev))
            x = torch.cat([img, model.embed(ids)], 0)
            if kind == 'prefill':
                g = harness.capture(lambda: model.prefill(x))
            else:
                _, ks, vs = model.prefill(x)
                cache = gemma.KVCache(ks, vs, BB_DECODE)

                def steps():
                    cache.rewind()
                    for t in range(BB_DECODE):
                        model.decode_step_cached(model.embed(dec[t]), cache)
                g = harness.capture(steps)
        calls = [g.replay]
    else:
        SW, M, N, Kd = 8, 800, 16384, 2048
        qw = torch.randint(-127, 128, (SW, N, Kd), generator=g, device=dev, dtype=torch.int8)
        qa = torch.randint(-127, 128, (M, Kd), generator=g, device=dev, dtype=torch.int8)
        acc = torch.empty(M, N, dtype=torch.int32, device=dev)
        calls = [lambda i=i: K.gemm_i8(qa, qw[i], acc) for i in range(SW)]
    for _ in range(reps):
        for c in calls:
            c()
    torch.cuda.synchronize()
    note(f'probe {kind}: {reps} x {len(calls)} calls')


def traced_classes(kind, seed):
    """harness.kernel_classes of the fly stages of `kind` ('chunk': one action chunk; 'backbone': the prefill and the 32
    decode steps), traced in a child process (`bench.py --classes kind`) on the same seeded setup: the device tracer then
    runs apart from the measurements, and a failure inside it costs only this record."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), '--classes', kind, '--seed', str(seed)]
    try:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=300)
    except subprocess.TimeoutExpired:
        return dict(error='tracer child timed out after 300 s')
    lines = [line for line in r.stdout.splitlines() if line.startswith('{')]
    if r.returncode != 0 or not lines:
        return dict(error=f'tracer child exited with status {r.returncode}')
    return json.loads(lines[-1])


def classes_child(kind, seed, dev):
    """--classes: the kernel classes of the fly stages of `kind`, as one JSON line on stdout."""
    import torch
    from yanlongvla_amd import gemma, harness, modules
    with torch.inference_mode():
        if kind == 'chunk':
            ks, vs, noise = expert_setup(seed, dev)
            model, _ = expert_policy('fly', seed, dev, ks, vs)

            def chunk():
                return model.sample_chunk(noise, CHUNK_STEPS)
            chunk()
            out = harness.kernel_classes(harness.capture(chunk), chunk)
        else:
            img, ids, dec = backbone_setup(seed, dev)
            model = gemma.make_policy(gemma.BackbonePolicy, dev, seed=seed + 1)
            modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, seed + 9, dev))
            x = torch.cat([img, model.embed(ids)], 0)
            state = {}

            def prefill():
                h, ks, vs = model.prefill(x)
                state.update(ks=ks, vs=vs)
                return h
            prefill()
            cache = gemma.KVCache(state['ks'], state['vs'], BB_DECODE)

            def decode():
                cache.rewind()
                return torch.cat([model.decode_step_cached(model.embed(dec[t]), cache) for t in range(BB_DECODE)], 0)
            out = {'prefill': harness.kernel_classes(harness.capture(prefill), prefill)}
            prefill()
            out['decode_32_tokens'] = harness.kernel_classes(harness.capture(decode), decode)
    torch.cuda.synchronize()
    note(f'kernel classes of the {kind} traced')
    print(json.dumps(out), flush=True)


def note(msg):
    """Progress line of a finished stage, on stderr (the JSON result line stays alone on stdout)."""
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({'error': f'--gpus {args.gpus}: this benchmark runs on one GPU only; the path has no multi-GPU '
                                   'implementation (row-split sharding is described in the design notes)'}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.probe:
        import torch
        from yanlongvla_amd import _lib
        _lib.lib()
        torch.cuda.set_device(0)
        probe(args.probe, args.probe_reps, torch.device('cuda:0'))
        return
    if args.classes:
        import torch
        from yanlongvla_amd import _lib
        _lib.lib()
        torch.cuda.set_device(0)
        classes_child(args.classes, args.seed, torch.device('cuda:0'))
        return
    import torch
    from yanlongvla_amd import _lib
    _lib.lib()
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    nl = args.layers
    L = make_stream(nl, args.seed, dev)
    gx = torch.Generator(device=dev).manual_seed(args.seed + 1)
    x = torch.randn(1, N_DIM, generator=gx, device=dev).half()
    S = Stream(L, x)
    S.step()
    torch.cuda.synchronize()
    err = check_against_oracle(L, S)
    if not err < 2e-3:
        raise SystemExit(f'decode-GEMV output differs from the oracle: relative L2 {err}')
    note(f'layer stream checked against the oracle (relative L2 {err:.2e})')

    ms_step = timed(S.step, args.steps, args.warmup, args.warmup_seconds)
    ms_gemv = timed(S.gemv, args.steps, args.warmup, 0.5)
    byts = nl * PACKED_BYTES
    achieved = byts / (ms_gemv * 1e-3) / 1e9
    note(f'layer stream timed: {ms_step:.4f} ms per step, {ms_gemv:.4f} ms per decode-GEMV launch')
    # single-layer latency (one layer, one token: rotation, decode-GEMV, rotation), HIP graph replays
    L1 = dict(L, tlut=L['tlut'][:1], row_scale=L['row_scale'][:1], sv=L['sv'][:1], wdev=L['wdev'][:L['per']])
    S1 = Stream(L1, x, fused=False)            # a single layer runs the latency plan (128 workgroups) and a separate rotation
    lat_med, lat_p95 = graph_latency(S1.step)
    am_med, am_p95 = graph_latency(S1.step, replays=50, warmup=5, per_graph=100)
    # the same layer in one launch (tcq_layer_f16: rotation, decode-GEMV and rotation in one kernel), equal bit for bit
    from yanlongvla_amd import kernels as K
    y1 = torch.empty(1, M_DIM, dtype=torch.float16, device=dev)
    z1 = torch.empty(1, M_DIM, dtype=torch.float32, device=dev)
    counter = torch.zeros(1, dtype=torch.int32, device=dev)

    def one_launch():
        K.layer_f16(x, L1['su'], L1['wdev'], L1['tlut'][0], L1['row_scale'][0], L1['sv'][0], None, y1, z1, counter)
    one_launch()
    S1.step()
    torch.cuda.synchronize()
    if not torch.equal(y1, S1.y[0]):
        raise SystemExit('the one-launch layer differs from the three-launch chain')
    one_med, one_p95 = graph_latency(one_launch)
    one_am_med, one_am_p95 = graph_latency(one_launch, replays=50, warmup=5, per_graph=100)

    # and in two launches (tcq_pre_gemv_f16: input rotation and decode-GEMV in one kernel; then the output rotation, tcq_post)
    def two_launch():
        K.pre_gemv_f16(x, L1['su'], L1['wdev'], L1['tlut'][0], L1['row_scale'][0], S1.z[0])
        K.post(S1.z[0], None, None, L1['sv'][0], None, S1.y[0])
    S1.y.zero_()
    two_launch()
    torch.cuda.synchronize()
    if not torch.equal(y1, S1.y[0]):
        raise SystemExit('the two-launch layer differs from the three-launch chain')
    two_med, two_p95 = graph_latency(two_launch)
    two_am_med, two_am_p95 = graph_latency(two_launch, replays=50, warmup=5, per_graph=100)
    note(f'single-layer latency timed: {lat_med:.4f} ms per graph replay (three launches), {two_med:.4f} (two), '
         f'{one_med:.4f} (one)')
    cpu = None if args.no_cpu else cpu_baseline(L, x, args.cpu_seconds)
    if cpu:
        note(f'CPU baseline timed: {cpu["value"]} {cpu["unit"]}')
    ops = None
    if not args.no_ops:
        ops = {'rht_bf16': rht_figures(dev, args.seed), 'w8a8_gemm_K2048_N16384': gemm_figures(dev, args.seed)}
        note('RHT and W8A8 GEMM shapes timed')
        if not args.no_cpu:
            ops['rht_bf16']['cpu_baseline'] = rht_cpu_baseline(args.seed, args.cpu_seconds / 2)
            ops['w8a8_gemm_K2048_N16384']['cpu_baseline'] = gemm_cpu_baseline(args.seed, args.cpu_seconds / 2)
            note('RHT and W8A8 GEMM CPU baselines timed')
    chunk = None
    if not args.no_chunk:
        del S1, L1
        chunk, keep, setup = action_chunk(args, dev)
        if not all(chunk['bitexact_vs_reference_runtime'].values()):
            raise SystemExit(f'action chunk differs from the reference runtime: {chunk["bitexact_vs_reference_runtime"]}')
        note(f'action chunk timed: {chunk["ms_per_chunk"]} ms (fly)')
        chunk['cpu_baseline'] = None if args.no_cpu else chunk_cpu_baseline(keep, setup, args.cpu_seconds)
        if chunk['cpu_baseline']:
            note('action chunk CPU baseline timed')
    out = {
        'metric': 'TCQ-2bit decode-GEMV GB/s (% HBM peak) + ms per action chunk, 1 GPU',
        'value': round(byts / (ms_step * 1e-3) / 1e9, 2),
        'unit': 'GB/s',
        'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'warmup_seconds_min': args.warmup_seconds,
        'ms_per_step': round(ms_step, 5),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'fp16',
        'data': 'synthetic (seeded uniform-random packed trellis words, N(0,1) FP16 tables, random signs, N(0,1) FP16 input)',
        'config': {'workload': f'tcq2 decode-GEMV layer stream: {nl} distinct 2048x2048 layers, batch 1, FP16 activations, '
                               'FP16 512x2 codebook, L=16 K=2 V=2, input and output block-Walsh rotations',
                   'layers': nl, 'm': M_DIM, 'n': N_DIM, 'tokens': 1, 'packed_bytes_per_step': byts},
        'hbm_frac': round(byts / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        'roofline': {'bound': 'hbm', 'kernel': 'k_gemv_f16<16, 4, 1, 2, 1, 1024, true, tcq_gemv_post_layer, 2> (layer stream, output rotation fused)', 'achieved': round(achieved, 2), 'peak': HBM_PEAK_GBS,
                     'unit': 'GB/s', 'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': traffic_from_profile(nl),
                     'ms_per_launch': round(ms_gemv, 5), 'bytes_per_launch': byts},
        'single_layer_ms': {'kernels': 'tcq_pre_gemv_f16 + tcq_post (two launches: input rotation and decode-GEMV, '
                                       'then the output rotation)',
                            'graph_replay_median': round(two_med, 5), 'graph_replay_p95': round(two_p95, 5),
                            'per_step_in_100_step_graph_median': round(two_am_med, 5),
                            'per_step_in_100_step_graph_p95': round(two_am_p95, 5),
                            'one_launch': {'kernel': 'tcq_layer_f16 (input rotation, decode-GEMV, output rotation)',
                                           'graph_replay_median': round(one_med, 5), 'graph_replay_p95': round(one_p95, 5),
                                           'per_step_in_100_step_graph_median': round(one_am_med, 5),
                                           'per_step_in_100_step_graph_p95': round(one_am_p95, 5)},
                            'three_launches': {'kernels': 'tcq_pre_h16 + tcq_gemv_f16 + tcq_postg',
                                               'graph_replay_median': round(lat_med, 5), 'graph_replay_p95': round(lat_p95, 5),
                                               'per_step_in_100_step_graph_median': round(am_med, 5),
                                               'per_step_in_100_step_graph_p95': round(am_p95, 5)},
                            'one_two_and_three_launches_equal': True},
        'max_rel_l2_vs_oracle': err,
        'cpu_baseline': cpu,
        'action_chunk': chunk,
        'ops': ops,
    }
    if not args.no_backbone:
        out['backbone'] = backbone(args, dev)
        note('backbone timed')
        if not all(out['backbone']['bitexact_vs_reference_runtime'].values()):
            raise SystemExit(f'backbone differs from the reference runtime: {out["backbone"]["bitexact_vs_reference_runtime"]}')
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
