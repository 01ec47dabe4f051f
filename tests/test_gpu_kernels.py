"""GPU parity of the HIP kernels against the CPU oracle (and, through it, the reference's own arithmetic): integer and
bit-pattern outputs bit-exact, the FP16-table float path within relative L2 2e-3 of the FP32/FP64 reference."""
import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'


@pytest.fixture(scope='module', autouse=True)
def _lib():
    from yanlongvla_amd import _lib
    _lib.lib()
    torch.cuda.init()


def T(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def layer_from(golden, tag):
    t = {k: golden[f'{tag}_{k}'] for k in ('bits', 'tlut', 'row_scale', 'su', 'sv')}
    bias = golden[f'{tag}_bias'] if f'{tag}_bias' in golden.files else None
    return O.Layer(tag, t, bias=bias)


def dev_layer(L):
    return dict(bits=T(L.bits), tlut=T(L.tlut.view(np.int16)), row_scale=T(L.row_scale.view(np.int16)), su=T(L.su), sv=T(L.sv))


def bits_of(t):
    return t.cpu().numpy().view(np.uint32 if t.element_size() == 4 else np.uint16)


# -------------------------------------------------------------------------------------------------------------------- snap
@pytest.mark.parametrize('tag', ['l0', 'l1', 'l2', 'l3', 'snap_neg', 'snap_tiny'])
def test_snap_bitexact(golden, tag):
    from yanlongvla_amd import kernels as K
    tl, rsc = golden[f'{tag}_tlut'], golden[f'{tag}_row_scale']
    t8, rs, g = K.snap(T(tl.view(np.int16)), T(rsc.view(np.int16)))
    assert np.array_equal(t8.cpu().numpy(), golden[f'{tag}_t8'])
    assert np.array_equal(bits_of(rs), golden[f'{tag}_rs'].view(np.uint32))
    assert bits_of(g)[0] == golden[f'{tag}_gain'].view(np.uint32)


# ------------------------------------------------------------------------------------------------------------------ decode
@pytest.mark.parametrize('m,n,seed', [(32, 48, 0), (48, 80, 1), (256, 1024, 2), (2048, 2048, 3), (1024, 4096, 4)])
def test_decode_i8_and_f16_bitexact(m, n, seed):
    from yanlongvla_amd import kernels as K
    L = O.random_layer(m, n, seed)
    d = dev_layer(L)
    t8, rs, _ = K.snap(d['tlut'], d['row_scale'])
    assert np.array_equal(t8.cpu().numpy(), L.t8)
    out = torch.empty(m, n, dtype=torch.int8, device=DEV)
    K.decode(d['bits'], t8, out)
    st = L.states()
    ref8 = O.lookup(st, L.t8.astype(np.int16)).astype(np.int8)
    assert np.array_equal(out.cpu().numpy(), ref8)
    out.fill_(77)
    K.decode_words(K.repack(d['bits'], m, n), t8, out)                   # the same bytes from the repacked words
    assert np.array_equal(out.cpu().numpy(), ref8)
    out16 = torch.empty(m, n, dtype=torch.int16, device=DEV)
    K.decode_f16(d['bits'], d['tlut'], out16)
    ref16 = O.lookup(st, L.tlut.astype(np.float32)).astype(np.float16)
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), ref16.view(np.uint16))


@pytest.mark.parametrize('tag', ['l0', 'l1', 'l2', 'l3'])
def test_decode_golden(golden, tag):
    from yanlongvla_amd import kernels as K
    L = layer_from(golden, tag)
    d = dev_layer(L)
    t8 = T(golden[f'{tag}_t8'])
    out = torch.empty(L.m, L.n, dtype=torch.int8, device=DEV)
    K.decode(d['bits'], t8, out)
    assert np.array_equal(out.cpu().numpy(), golden[f'{tag}_w8'])
    out.fill_(77)
    K.decode_words(K.repack(d['bits'], L.m, L.n), t8, out)
    assert np.array_equal(out.cpu().numpy(), golden[f'{tag}_w8'])


# -------------------------------------------------------------------------------------------------------------------- RHT
RHT_CASES = [(1, 1), (3, 16), (2, 48), (5, 80), (2, 20), (1, 1024), (16, 2048), (50, 4096), (3, 8192), (16, 16384), (4, 1152), (3, 4304),
             (800, 1024), (800, 16384)]


@pytest.mark.parametrize('M,n', RHT_CASES)
@pytest.mark.parametrize('xdt', [torch.bfloat16, torch.float32, torch.float16])
def test_rht_bitexact(M, n, xdt):
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(M * 7 + n)
    x = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(xdt)
    su = np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8)
    y = torch.empty(M, n, dtype=torch.float32, device=DEV)
    K.rht(x.to(DEV), T(su), y)
    ref = O.fwht(x.float().numpy() * su.astype(np.float32))
    assert np.array_equal(bits_of(y), ref.view(np.uint32))
    yb = torch.empty(M, n, dtype=torch.bfloat16, device=DEV)
    K.rht(x.to(DEV), T(su), yb)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), O.bf16_bits(ref))


@pytest.mark.parametrize('M,n,off', [(3, 4096, 32), (5, 16384, 32), (4, 2048, 32), (3, 8192, 1)])
def test_rht_strided_rows_f16_out(M, n, off):
    """Rows inside wider buffers (ldx = n + 64, ldy = n + 32) and FP16 output; off = 1 starts the rows off 16-byte
    alignment, which the aligned register paths must leave to the LDS engine."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(n + off)
    xf = rng.standard_normal((M, n + 64)).astype(np.float32)
    xb = torch.from_numpy(xf).bfloat16()
    su = np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8)
    x = xb.to(DEV)[:, off:off + n]
    yfull = torch.zeros(M, n + 32, dtype=torch.float16, device=DEV)
    K.rht(x, T(su), yfull[:, :n])
    ref = O.fwht(xb[:, off:off + n].float().numpy() * su.astype(np.float32))
    assert np.array_equal(yfull[:, :n].cpu().numpy().view(np.uint16), ref.astype(np.float16).view(np.uint16))
    assert not yfull[:, n:].any()


def fp16_tie_weight(n):
    """A value w whose product with c = float32(1/sqrt(n)), rounded to FP32, is an exact FP16 tie while the exact product is
    not: FP32-then-FP16 rounding (the definition) and a single rounding of the exact product to FP16 then differ."""
    c = np.float32(1.0 / np.sqrt(n))
    w = (1.0 + np.arange(1, 1 << 20) * 2.0 ** -20).astype(np.float32)
    p = w * c
    h = p.astype(np.float16)
    half_ulp = np.spacing(np.abs(h)).astype(np.float64) / 2
    tie = np.abs(p.astype(np.float64) - h.astype(np.float64)) == half_ulp
    single = (w.astype(np.float64) * np.float64(c)).astype(np.float16)
    cand = w[tie & (single != h)]
    assert cand.size, n
    return cand[0]


@pytest.mark.parametrize('n', [2048, 8192])
def test_rht_fp16_output_rounds_through_fp32(n):
    """Every output of a one-hot row is w * c: at an FP16 tie of the FP32 product the FP16 output must round that FP32 value
    (half-even), not the exact product (a fused multiply-convert would)."""
    from yanlongvla_amd import kernels as K
    w = fp16_tie_weight(n)
    x = np.zeros((2, n), dtype=np.float32)
    x[:, 0] = w
    y = torch.empty(2, n, dtype=torch.float16, device=DEV)
    K.rht(T(x), None, y)
    ref = O.fwht(x).astype(np.float16)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize('M,n', [(1, 1024), (16, 2048), (50, 4096)])
def test_rht_vs_dense_hadamard(M, n):
    """C1 contract: FP32 result within 1e-3 relative of a dense-Hadamard FP64 reference (closed form, not the oracle)."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(n)
    x = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).bfloat16()
    su = np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8)
    y = torch.empty(M, n, dtype=torch.float32, device=DEV)
    K.rht(x.to(DEV), T(su), y)
    H = torch.ones(1, 1, dtype=torch.float64)
    while H.shape[0] < n:
        H = torch.cat((torch.cat((H, H), 1), torch.cat((H, -H), 1)), 0)
    ref = (x.double() * torch.from_numpy(su).double()) @ H / np.sqrt(n)
    err = (y.cpu().double() - ref).norm() / ref.norm()
    assert err < 1e-3


@pytest.mark.parametrize('M,n', [(800, 16384), (800, 4096), (16, 4304)])
def test_rht_involution_full_size(M, n):
    """Size-independent property at the full C1 size: the normalised transform is its own inverse, and it preserves norms."""
    from yanlongvla_amd import kernels as K
    x = torch.randn(M, n, device=DEV)
    y = torch.empty_like(x)
    z = torch.empty_like(x)
    K.rht(x, None, y)
    K.rht(y, None, z)
    assert (z - x).norm() / x.norm() < 1e-5
    assert torch.allclose(y.norm(dim=1), x.norm(dim=1), rtol=1e-4)


# ------------------------------------------------------------------------------------------------------------ pre / post
@pytest.mark.parametrize('M,K', [(1, 48), (3, 80), (2, 20), (10, 1024), (16, 2048), (50, 4096), (7, 16384), (300, 2048),
                                 (4, 1152), (800, 4096)])
@pytest.mark.parametrize('xdt', [torch.bfloat16, torch.float32])
def test_pre_bitexact(M, K, xdt):
    from yanlongvla_amd import kernels as Kk
    rng = np.random.default_rng(M + K)
    x = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).to(xdt)
    if M > 2:
        x[2] = 0                                  # all-zero token -> scale 1
    su = np.where(rng.integers(0, 2, K) > 0, 1, -1).astype(np.int8)
    q = torch.empty(M, K, dtype=torch.int8, device=DEV)
    q4 = torch.empty(K // 4, M, dtype=torch.int32, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    Kk.pre(x.to(DEV), T(su), q=q, q4=q4, scale=s)
    qr, sr = O.quantize_tokens(O.fwht(x.float().numpy() * su.astype(np.float32)))
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(bits_of(s), sr[:, 0].view(np.uint32))
    assert np.array_equal(q4.cpu().numpy(), O.q4_layout(qr))


@pytest.mark.parametrize('M,N', [(1, 16), (3, 48), (2, 20), (10, 256), (16, 2048), (50, 4096), (5, 16384), (300, 1024),
                                 (2, 4304), (800, 2048), (7, 1024), (64, 256), (1, 2048)])
def test_post_bitexact(M, N):
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(M * N)
    acc = rng.integers(-2 ** 20, 2 ** 20, size=(M, N + 8)).astype(np.int32)
    s = (rng.random(M) + 0.5).astype(np.float32)
    rs = (rng.random(N + 8) * 1e-3).astype(np.float32)
    sv = np.where(rng.integers(0, 2, N + 8) > 0, 1, -1).astype(np.int8)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    col0 = 8 if M % 2 else 0
    for with_bias in (False, True):
        y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        K.post(T(acc), T(s), T(rs[col0:col0 + N].copy()), T(sv[col0:col0 + N].copy()), T(bias) if with_bias else None, y, col0=col0)
        z = (acc[:, col0:col0 + N].astype(np.float32) * s[:, None]) * rs[None, col0:col0 + N]
        ref = O.post_bf16(z, sv[col0:col0 + N], bias if with_bias else None)
        assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)
    # FP32 accumulators (already scaled), FP32 and FP16 outputs
    zf = (rng.standard_normal((M, N)) * 0.3).astype(np.float32)
    for ydt in (torch.float32, torch.float16):
        y = torch.empty(M, N, dtype=ydt, device=DEV)
        K.post(T(zf), None, None, T(sv[:N].copy()), None, y)
        ref = O.fwht(zf) * sv[:N].astype(np.float32)
        if ydt == torch.float32:
            assert np.array_equal(bits_of(y), ref.view(np.uint32))
        else:
            assert np.array_equal(y.cpu().numpy().view(np.uint16), ref.astype(np.float16).view(np.uint16))
    # BF16 accumulators (scaled by the row scale only), BF16 output
    ab = torch.from_numpy((rng.standard_normal((M, N)) * 100).astype(np.float32)).bfloat16()
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    K.post(ab.to(DEV), None, T(rs[:N].copy()), T(sv[:N].copy()), None, y)
    ref = O.post_bf16(ab.float().numpy() * rs[None, :N], sv[:N])
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize('tag', ['l0', 'l1', 'l2', 'l3'])
@pytest.mark.parametrize('dt', ['f32', 'bf16'])
def test_w2a8_layer_golden(golden, tag, dt):
    """pre -> decode -> exact INT32 product -> post against the reference's own W2A8 outputs, bit for bit."""
    from yanlongvla_amd import kernels as K
    L = layer_from(golden, tag)
    d = dev_layer(L)
    t8, rs, _ = K.snap(d['tlut'], d['row_scale'])
    x = golden[f'{tag}_x_{dt}']
    xt = torch.from_numpy(x).view(torch.bfloat16) if dt == 'bf16' else torch.from_numpy(x)
    M = xt.shape[0]
    q = torch.empty(M, L.n, dtype=torch.int8, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    K.pre(xt.to(DEV), d['su'], q=q, scale=s)
    w8 = torch.empty(L.m, L.n, dtype=torch.int8, device=DEV)
    K.decode(d['bits'], t8, w8)
    acc = O.int_matmul(q.cpu().numpy(), w8.cpu().numpy())       # exact products; the INT8 GEMM kernel is tested on its own
    y = torch.empty(M, L.m, dtype=torch.bfloat16, device=DEV)
    bias = None if L.bias is None else T(L.bias)
    K.post(T(acc), s, rs, d['sv'], bias, y)
    assert np.array_equal(y.view(torch.int16).cpu().numpy(), golden[f'{tag}_y_{dt}_a8_int8'])


# ------------------------------------------------------------------------------------------------------ FP16-table GEMV
def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# latency plan (<= 2048 tile rows per batch: one tile row per workgroup, 4 / 8 / 16 waves splitting the chunks) and the
# stream plan (row groups per wave; one workgroup per layer from 256 layers on)
@pytest.mark.parametrize('m,n,M,nl', [(2048, 2048, 1, 1), (2048, 2048, 4, 3), (48, 80, 1, 2), (256, 1024, 16, 1),
                                      (1024, 4096, 1, 2), (4096, 1024, 2, 1), (64, 1152, 3, 2), (512, 512, 2, 1),
                                      (1024, 16384, 1, 1), (2048, 2048, 1, 17), (128, 256, 1, 300), (64, 1152, 3, 600)])
def test_gemv_f16_layer(m, n, M, nl):
    """Dense-table layer: pre_h16 -> fused decode-GEMV -> post, against reference_linear(table='fp16', a8=False),
    rel L2 <= 2e-3."""
    from yanlongvla_amd import kernels as K
    layers = [O.random_layer(m, n, 100 + i) for i in range(nl)]
    for L in layers[1:]:
        L.su = layers[0].su                              # a batch shares the input rotation (su depends only on n)
    rng = np.random.default_rng(m + n + M)
    x = rng.standard_normal((M, n)).astype(np.float16)
    xd = T(x.view(np.int16)).view(torch.float16)
    h16 = torch.empty(M, n, dtype=torch.float16, device=DEV)
    hs = torch.empty(M, dtype=torch.float32, device=DEV)
    dl = [dev_layer(L) for L in layers]
    K.pre_h16(xd, dl[0]['su'], h16, hs)
    zs = [torch.empty(M, m, dtype=torch.float32, device=DEV) for _ in layers]
    wdevs = [K.repack(d['bits'], m, n) for d in dl]
    desc = K.gemv_descriptors([(w, d['tlut'], d['row_scale'], z) for w, d, z in zip(wdevs, dl, zs)])
    K.gemv_f16(desc, h16, hs, m, n)
    for L, d, z in zip(layers, dl, zs):
        y = torch.empty(M, m, dtype=torch.float32, device=DEV)
        K.post(z, None, None, d['sv'], None, y)
        ref = O.reference_linear(x.astype(np.float32), L, a8=False, table='fp16', out_dtype='f32')
        assert rel_l2(y.cpu().numpy(), ref) < 2e-3
        # accumulator before the output rotation
        h = O.fwht(x.astype(np.float32) * L.su.astype(np.float32))
        zr = (h.astype(np.float64) @ O.lookup(L.states(), L.tlut.astype(np.float32)).astype(np.float64).T) * \
            L.row_scale.astype(np.float64)[None, :]
        assert rel_l2(z.cpu().numpy(), zr) < 2e-3
        y16 = torch.empty(M, m, dtype=torch.float16, device=DEV)
        K.post(z, None, None, d['sv'], None, y16)
        assert rel_l2(y16.cpu().float().numpy(), ref) < 2e-3


# one launch of a whole layer: the latency plan's split (4 / 8 / 16 waves per tile row), non-power-of-two widths (block
# Walsh), several tokens, every input and output type
@pytest.mark.parametrize('m,n,M,xdt,ydt', [(2048, 2048, 1, torch.float16, torch.float16), (2048, 2048, 4, torch.bfloat16, torch.float32),
                                           (1024, 4096, 1, torch.float32, torch.bfloat16), (4096, 1024, 2, torch.float16, torch.float16),
                                           (64, 1152, 3, torch.float16, torch.float32), (1536, 512, 1, torch.bfloat16, torch.bfloat16),
                                           (256, 16384, 1, torch.float16, torch.float16), (1024, 1024, 16, torch.float32, torch.bfloat16),
                                           (2048, 2048, 16, torch.bfloat16, torch.float16)])
def test_layer_f16_one_launch(m, n, M, xdt, ydt):
    """tcq_layer_f16 equals the three-launch chain pre_h16 -> gemv_f16 -> post bit for bit (y and z), twice in a row on
    different inputs (the second call finds the counter the first left at zero), and is within 2e-3 of the oracle's
    reference_linear(table='fp16', a8=False); tcq_pre_gemv_f16 gives the same z."""
    from yanlongvla_amd import kernels as K
    L = O.random_layer(m, n, 300 + m + M)
    d = dev_layer(L)
    bias = torch.randn(m, device=DEV) * 0.1
    wdev = K.repack(d['bits'], m, n)
    z = torch.empty(M, m, dtype=torch.float32, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    rng = np.random.default_rng(m + n)
    for call in range(2):
        x = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).to(DEV).to(xdt)
        y = torch.empty(M, m, dtype=ydt, device=DEV)
        K.layer_f16(x, d['su'], wdev, d['tlut'], d['row_scale'], d['sv'], bias, y, z, counter)
        h16 = torch.empty(M, n, dtype=torch.float16, device=DEV)
        hs = torch.empty(M, dtype=torch.float32, device=DEV)
        K.pre_h16(x, d['su'], h16, hs)
        z3 = torch.empty(M, m, dtype=torch.float32, device=DEV)
        K.gemv_f16(K.gemv_descriptors([(wdev, d['tlut'], d['row_scale'], z3)]), h16, hs, m, n)
        y3 = torch.empty(M, m, dtype=ydt, device=DEV)
        K.post(z3, None, None, d['sv'], bias, y3)
        assert torch.equal(z, z3), call
        z2 = torch.full((M, m), float('nan'), dtype=torch.float32, device=DEV)
        K.pre_gemv_f16(x, d['su'], wdev, d['tlut'], d['row_scale'], z2)
        assert torch.equal(z2, z3), call
        assert torch.equal(y.view(torch.int16) if ydt != torch.float32 else y, y3.view(torch.int16) if ydt != torch.float32 else y3), call
        assert int(counter.item()) == 0
        ref = O.reference_linear(x.float().cpu().numpy(), L, a8=False, table='fp16', out_dtype='f32') + bias.cpu().numpy()
        assert rel_l2(y.float().cpu().numpy(), ref) < 2e-3


def test_layer_f16_graph_replays():
    """A captured one-launch layer replays to the eager result several times, with eager calls in between."""
    from yanlongvla_amd import kernels as K
    L = O.random_layer(2048, 2048, 77)
    d = dev_layer(L)
    wdev = K.repack(d['bits'], 2048, 2048)
    x = torch.randn(1, 2048, device=DEV).half()
    z = torch.empty(1, 2048, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    y = torch.empty(1, 2048, dtype=torch.float16, device=DEV)
    step = lambda: K.layer_f16(x, d['su'], wdev, d['tlut'], d['row_scale'], d['sv'], None, y, z, counter)
    step()
    eager = y.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(3):
            step()
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager) and int(counter.item()) == 0
        step()
        assert torch.equal(y, eager)


@pytest.mark.parametrize('K,M,xdt', [(256, 1, torch.float16), (1024, 3, torch.bfloat16), (2048, 1, torch.float16),
                                     (16384, 2, torch.float32), (1152, 2, torch.float16), (2048, 5, torch.bfloat16),
                                     (1024, 64, torch.float32), (2048, 65, torch.float16)])
def test_pre_h16_bitexact(K, M, xdt):
    """The float path's input rotation (no-transpose engine for up to 64 rows of 1024 / 2048, register engine for other
    power-of-two rows, LDS engine otherwise) against the oracle:
    h = fwht(x * su), hscale = 2^e with amax / 2^e in [2^14, 2^15), h16 = FP16(h / hscale), bit for bit."""
    from yanlongvla_amd import kernels as K_
    rng = np.random.default_rng(K + M)
    x32 = rng.standard_normal((M, K)).astype(np.float32)
    su = (rng.integers(0, 2, K) * 2 - 1).astype(np.int8)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    h16 = torch.empty(M, K, dtype=torch.float16, device=DEV)
    hs = torch.empty(M, dtype=torch.float32, device=DEV)
    K_.pre_h16(x, T(su), h16, hs)
    h = O.fwht(x.float().cpu().numpy() * su.astype(np.float32))
    for t in range(M):
        e = int(np.frexp(np.abs(h[t]).max())[1]) - 15
        assert hs[t].item() == 2.0 ** e
        want = np.ldexp(h[t], -e).astype(np.float16).view(np.uint16)
        assert np.array_equal(h16[t].cpu().numpy().view(np.uint16), want), t


def test_gemv_f16_deterministic():
    from yanlongvla_amd import kernels as K
    L = O.random_layer(512, 2048, 7)
    d = dev_layer(L)
    h16 = torch.randn(1, 2048, device=DEV).half()
    hs = torch.ones(1, device=DEV)
    w = K.repack(d['bits'], 512, 2048)
    z1, z2 = torch.empty(1, 512, device=DEV), torch.empty(1, 512, device=DEV)
    K.gemv_f16(K.gemv_descriptors([(w, d['tlut'], d['row_scale'], z1)]), h16, hs, 512, 2048)
    K.gemv_f16(K.gemv_descriptors([(w, d['tlut'], d['row_scale'], z2)]), h16, hs, 512, 2048)
    assert torch.equal(z1, z2)


@pytest.mark.parametrize('nl,M,m,n', [(300, 1, 512, 1024), (260, 3, 256, 512), (3, 4, 2048, 2048), (2, 1, 8192, 1024),
                                      (5, 16, 256, 512)])
@pytest.mark.parametrize('ydt', [torch.float16, torch.bfloat16, torch.float32])
def test_gemv_post_fused_equals_unfused(nl, M, m, n, ydt):
    """tcq_gemv_f16_post == tcq_gemv_f16 then tcq_post (FP32 z), with and without bias: bit for bit when the unfused launch
    also runs the layer-stream plan (>= 256 layers), else within the summation-order difference of its latency plan."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(nl + M + m)
    layers = [dev_layer(O.random_layer(m, n, 50 + i, bias=i % 2 == 1)) for i in range(nl)]
    h16 = T(rng.standard_normal((M, n)).astype(np.float16))
    hs = T(np.full(M, 0.5, np.float32))
    ws = [K.repack(d['bits'], m, n) for d in layers]
    zs = [torch.empty(M, m, device=DEV) for _ in layers]
    K.gemv_f16(K.gemv_descriptors([(w, d['tlut'], d['row_scale'], z) for w, d, z in zip(ws, layers, zs)]), h16, hs, m, n)
    ys = [torch.empty(M, m, dtype=ydt, device=DEV) for _ in layers]
    biases = [T(rng.standard_normal(m).astype(np.float32)) if i % 2 else None for i in range(nl)]
    desc = K.gemv_post_descriptors([(w, d['tlut'], d['row_scale'], d['sv'], b, y) for w, d, b, y in zip(ws, layers, biases, ys)])
    K.gemv_f16_post(desc, h16, hs, m, n, ydt)
    for z, d, b, y in zip(zs, layers, biases, ys):
        ref = torch.empty(M, m, dtype=ydt, device=DEV)
        K.post(z, None, None, d['sv'], b, ref)
        if nl >= 256:
            assert torch.equal(y.view(torch.int16) if ydt != torch.float32 else y, ref.view(torch.int16) if ydt != torch.float32 else ref)
        else:
            assert ((y.double() - ref.double()).norm() / ref.double().norm()).item() < (2e-3 if ydt != torch.float32 else 1e-6)


def test_layer_stream_2048_against_the_oracle():
    """The benchmarked pass itself against the oracle: 256 distinct 2048 x 2048 layers (one FP16 scale per layer, N(0, 1)
    FP16 tables, random signs), one FP16 token x ~ N(0, 1), input rotation by pre_h16, then one gemv_f16_post launch over
    the whole stream (the layer-stream plan, output rotation fused, FP16 y). Every 8th layer and the last one are checked
    against the oracle's reference_linear(table='fp16', a8=False) (tcq_format.py:125-148): relative L2 <= 2e-3."""
    from yanlongvla_amd import kernels as K
    nl, m, n = 256, 2048, 2048
    layers = [O.random_layer(m, n, 900 + i) for i in range(nl)]
    su = layers[0].su
    for L in layers:                                   # one stream shares the input signs (one input rotation)
        L.su = su
    devs = [dev_layer(L) for L in layers]
    x = np.random.default_rng(901).standard_normal((1, n)).astype(np.float16)
    h16 = torch.empty(1, n, dtype=torch.float16, device=DEV)
    hs = torch.empty(1, dtype=torch.float32, device=DEV)
    K.pre_h16(T(x), T(su), h16, hs)
    ws = [K.repack(d['bits'], m, n) for d in devs]
    ys = [torch.empty(1, m, dtype=torch.float16, device=DEV) for _ in range(nl)]
    desc = K.gemv_post_descriptors([(w, d['tlut'], d['row_scale'], d['sv'], None, y) for w, d, y in zip(ws, devs, ys)])
    K.gemv_f16_post(desc, h16, hs, m, n, torch.float16)
    torch.cuda.synchronize()
    errs = {}
    for i in sorted(set(range(0, nl, 8)) | {nl - 1}):
        ref = O.reference_linear(x.astype(np.float32), layers[i], a8=False, table='fp16', out_dtype='f32')
        y = ys[i].float().cpu().numpy()
        errs[i] = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    worst = max(errs, key=errs.get)
    print(f'layer stream 256 x 2048^2: max rel L2 {errs[worst]:.2e} (layer {worst}) over {len(errs)} layers', flush=True)
    assert errs[worst] <= 2e-3, (worst, errs[worst])


# ------------------------------------------------------------------------------------------------------ batched epilogue
@pytest.mark.parametrize('M', [1, 10, 50])
def test_postg_matches_post_and_oracle(M):
    """q / k / v style segments sharing one INT32 accumulator row, plus separate FP32 accumulators, with bias and GELU."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(M)
    widths = [2048, 256, 256]
    lda = sum(widths)
    acc = rng.integers(-2 ** 20, 2 ** 20, size=(M, lda)).astype(np.int32)
    s = (rng.random(M) + 0.5).astype(np.float32)
    rs = (rng.random(lda) * 1e-3).astype(np.float32)
    sv = np.where(rng.integers(0, 2, lda) > 0, 1, -1).astype(np.int8)
    bias = (rng.standard_normal(lda) * 0.1).astype(np.float32)
    accd, sd = T(acc), T(s)
    ys, segs, c0 = [], [], 0
    for i, w in enumerate(widths):
        y = torch.empty(M, w, dtype=torch.bfloat16, device=DEV)
        segs.append((accd, c0, T(rs[c0:c0 + w].copy()), T(sv[c0:c0 + w].copy()), T(bias[c0:c0 + w].copy()) if i else None, y, i == 0))
        ys.append(y)
        c0 += w
    lut = K.gelu_table(DEV)
    desc = K.post_segments(segs, DEV)
    K.post_batched(desc, len(segs), torch.int32, torch.bfloat16, sd, M, max(widths), gelu_lut=lut)
    lut_np = lut.view(torch.int16).cpu().numpy().view(np.uint16)
    c0 = 0
    for i, (w, y) in enumerate(zip(widths, ys)):
        z = (acc[:, c0:c0 + w].astype(np.float32) * s[:, None]) * rs[None, c0:c0 + w]
        ref = O.post_bf16(z, sv[c0:c0 + w], bias[c0:c0 + w] if i else None)
        if i == 0:
            ref = lut_np[ref]
        assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), ref)
        c0 += w
    # FP32 accumulators of separate layers (the decode-GEMV outputs), FP32 outputs
    zs = [T((rng.standard_normal((M, 512)) * 0.2).astype(np.float32)) for _ in range(5)]
    svs = [np.where(rng.integers(0, 2, 512) > 0, 1, -1).astype(np.int8) for _ in range(5)]
    outs = [torch.empty(M, 512, dtype=torch.float32, device=DEV) for _ in range(5)]
    desc = K.post_segments([(z, 0, None, T(v), None, y, False) for z, v, y in zip(zs, svs, outs)], DEV)
    K.post_batched(desc, 5, torch.float32, torch.float32, None, M, 512)
    for z, v, y in zip(zs, svs, outs):
        ref = O.fwht(z.cpu().numpy()) * v.astype(np.float32)
        assert np.array_equal(bits_of(y), ref.view(np.uint32))


@pytest.mark.parametrize('M', [1, 7])
def test_postg_few_tokens_mixed_widths(M):
    """Device descriptors with a 2048-wide segment beside segments of other widths and an unaligned column offset: the
    few-token kernel rotates the aligned 2048 / 256 segments on its own engine and the rest on the LDS engine; every output
    equals the oracle's epilogue bit for bit."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(100 + M)
    widths, col0s, lda = [2048, 256, 1024, 300, 256], [0, 2048, 2304, 3328, 3629], 3900
    acc = (rng.standard_normal((M, lda)) * 0.3).astype(np.float32)
    sv = np.where(rng.integers(0, 2, lda) > 0, 1, -1).astype(np.int8)
    bias = (rng.standard_normal(lda) * 0.1).astype(np.float32)
    accd, segs, ys = T(acc), [], []
    for i, (w, c0) in enumerate(zip(widths, col0s)):
        y = torch.empty(M, w, dtype=torch.bfloat16, device=DEV)
        segs.append((accd, c0, None, T(sv[c0:c0 + w].copy()), T(bias[c0:c0 + w].copy()) if i % 2 else None, y, i == 2))
        ys.append(y)
    lut = K.gelu_table(DEV)
    desc = K.post_segments(segs, DEV)
    K.post_batched(desc, len(segs), torch.float32, torch.bfloat16, None, M, 2048, gelu_lut=lut)
    lut_np = lut.view(torch.int16).cpu().numpy().view(np.uint16)
    for i, (w, c0, y) in enumerate(zip(widths, col0s, ys)):
        ref = O.post_bf16(acc[:, c0:c0 + w], sv[c0:c0 + w], bias[c0:c0 + w] if i % 2 else None)
        if i == 2:
            ref = lut_np[ref]
        assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), ref), i


def test_bf16_conversion_of_every_exponent_and_payload():
    """FP32 -> BF16 of the kernels (round to nearest even, NaN -> 0x7fc0) over every high half-word with low halves at and
    around the rounding tie (0x7fff, 0x8000, 0x8001), the extremes and two payloads: infinities, subnormals, overflow to
    infinity and NaNs of every sign and payload. One-sided plain epilogue, FP32 in, BF16 out (a conversion only)."""
    from yanlongvla_amd import kernels as K
    hi = np.arange(65536, dtype=np.uint32) << 16
    lo = np.array([0x0000, 0x0001, 0x4000, 0x7fff, 0x8000, 0x8001, 0xc000, 0xffff], dtype=np.uint32)
    u = (hi[:, None] | lo[None, :]).reshape(64, -1)
    x = T(u.view(np.int32)).view(torch.float32)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    K.post(x, None, None, None, None, y)
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), O.bf16_bits(u.view(np.float32)))


def test_quantizer_at_rounding_ties():
    """The INT8 quantizer's quotient v / s (reciprocal + two corrections for scales in [2^-90, 2^90], IEEE division
    outside) against the oracle's FP32 division on rows built around the rounding ties: v = (k + 1/2) s moved by 0, +-1,
    +-2 ulp for every k in -127 .. 126, with the row maximum 127 s fixing s; row scales from 1e-36 to 1e36, on both sides
    of both ends of the reciprocal's range."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(17)
    rows = []
    for amax in (1e-36, 127 * 2.0 ** -90 * 0.999, 127 * 2.0 ** -90 * 1.001, 1e-20, 0.37, 1.0, 127.0, 3.3e11,
                 127 * 2.0 ** 90 * 0.999, 127 * 2.0 ** 90 * 1.001, 1e36):
        a = np.float32(amax)
        s = a / np.float32(127)
        k = np.arange(-127, 127, dtype=np.float32)
        base = ((k + np.float32(0.5)) * s).astype(np.float32)
        ties = np.concatenate([(base.view(np.int32) + d).view(np.float32) for d in (-2, -1, 0, 1, 2)])
        ties = ties[np.abs(ties) <= a]
        row = np.concatenate([[a], ties, (rng.uniform(-1, 1, 2048) * a).astype(np.float32)])[:2048]
        rows.append(np.pad(row, (0, 2048 - row.size)))
    x = np.stack(rows).astype(np.float32)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    sc = torch.empty(x.shape[0], device=DEV)
    K.quantize_rows(T(x), q, sc)
    qr, sr = O.quantize_tokens(x)
    assert np.array_equal(sc.cpu().numpy(), sr[:, 0])
    assert np.array_equal(q.cpu().numpy(), qr)


def test_rht_bf16_output_of_nan_and_inf_rows():
    """BF16 outputs of the rotation for rows holding a NaN (any payload), opposite infinities or one infinity, against the
    oracle: a NaN reaches every output of its row and converts to 0x7fc0 (the packed two-value conversion with its NaN
    rule); inf - inf gives NaN at half the positions of its row."""
    from yanlongvla_amd import kernels as K
    n = 1024
    x = np.zeros((4, n), np.float32)
    x[0, 5] = np.uint32(0x7f812345).view(np.float32)      # signalling-style payload
    x[1, 9] = np.uint32(0xffc00001).view(np.float32)      # negative quiet NaN with payload
    x[2, 0], x[2, 1] = np.inf, -np.inf
    x[3, 3] = np.inf
    y = torch.empty(4, n, dtype=torch.bfloat16, device=DEV)
    K.rht(T(x), None, y)
    b = y.view(torch.int16).cpu().numpy().view(np.uint16)
    assert (b[:2] == 0x7fc0).all()
    with np.errstate(invalid='ignore'):
        ref = O.bf16_bits(O.fwht(x))
    assert np.array_equal(b, ref)
    assert (b[2] == 0x7fc0).sum() == n // 2


def test_gelu_table_vs_cpu():
    """The device GELU table against PyTorch's CPU routine over all 65,536 BF16 inputs: NaN at the same inputs (NaN inputs,
    and -inf, whose x * (1 + tanh(..)) is -inf * 0). Measured on MI355X, the two routines differ at 4 other inputs, -5.0625
    .. -5.15625 (0xc0a2 .. 0xc0a5), where 1 + tanh(..) cancels: the CPU result is -0, the device's about -1.5e-7. At most
    4 entries may differ, all at inputs below -5, each by at most 2^-22 in absolute value. The fused kernels use the
    device table, as the reference does."""
    from yanlongvla_amd import kernels as K
    dev = K.gelu_table(DEV).cpu()
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    cpu = torch.nn.functional.gelu(allb, approximate='tanh')
    nan = torch.isnan(cpu)
    assert torch.equal(torch.isnan(dev), nan)
    db = dev.view(torch.int16).numpy().view(np.uint16).astype(np.int64)
    cb = cpu.view(torch.int16).numpy().view(np.uint16).astype(np.int64)
    diff = np.flatnonzero((db != cb) & ~nan.numpy())
    print(f'GELU table: {diff.size} of {int((~nan).sum())} non-NaN BF16 results differ between device and CPU '
          f'(inputs {[hex(int(i)) for i in diff]})', flush=True)
    assert diff.size <= 4, diff.size
    x, d, c = allb.float().numpy(), dev.float().numpy(), cpu.float().numpy()
    assert (x[diff] < -5).all() and (np.abs(d[diff] - c[diff]) <= 2.0 ** -22).all(), \
        [(hex(int(i)), hex(int(db[i])), hex(int(cb[i]))) for i in diff]


# ------------------------------------------------------------------------------------------------- small-M INT8 products
def _small_product_case(shapes, M, seed):
    """Layers of one group (same n, shared input signs), INT8 activations, expected z from the exact integer product."""
    from yanlongvla_amd import kernels as K
    n = shapes[0][1]
    layers = [O.random_layer(m, n, seed + i) for i, (m, _) in enumerate(shapes)]
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, size=(M, n)).astype(np.int8)
    if M > 3:
        q[3] = 0
    s = (rng.random(M) * 0.02 + 1e-3).astype(np.float32)
    ldz = sum(L.m for L in layers)
    ref = np.concatenate([(O.int_matmul(q, L.w8_reference()).astype(np.float32) * s[:, None]) * L.rs[None, :] for L in layers], 1)
    dev = [dev_layer(L) for L in layers]
    t8s = [K.snap(d['tlut'], d['row_scale'])[:2] for d in dev]
    return layers, dev, t8s, q, s, ldz, ref


@pytest.mark.parametrize('shapes,M', [([(2048, 1024)], 1), ([(2048, 1024), (256, 1024), (256, 1024)], 50),
                                      ([(1024, 2048)], 16), ([(4096, 1024), (4096, 1024)], 17), ([(1024, 4096)], 64),
                                      ([(64, 1152)], 33), ([(48, 80), (32, 80)], 5), ([(256, 16384)], 10),
                                      ([(4112, 1024), (2048, 1024)], 50),
                                      # streaming plan of the fused product (one token block, >= 4096 chunks): 16, 4, 2 and 1
                                      # waves per tile row
                                      ([(2048, 16384)], 1), ([(16384, 2048)], 16), ([(8192, 2048)] * 4, 1),
                                      ([(65536, 1024)], 1)])
def test_gemm_tcq_and_w8_bitexact(shapes, M):
    """Fused decode + INT8 product and the INT8-resident product against the oracle, FP32 bits equal (exact int32 sums)."""
    from yanlongvla_amd import kernels as K
    layers, dev, t8s, q, s, ldz, ref = _small_product_case(shapes, M, 31 * M + len(shapes))
    n = layers[0].n
    qd, sd = T(q), T(s)
    z = torch.full((M, ldz), float('nan'), device=DEV)
    z2 = torch.full((M, ldz), float('nan'), device=DEV)
    wdevs = [K.repack(d['bits'], L.m, n) for L, d in zip(layers, dev)]
    w8s = []
    for L, d, (t8, _) in zip(layers, dev, t8s):
        w = torch.empty(L.m, n, dtype=torch.int8, device=DEV)
        K.decode(d['bits'], t8, w)
        w8s.append(w)
    cols, c0 = [], 0
    for L in layers:
        cols.append(c0)
        c0 += L.m
    K.gemm_tcq_segments([(w, t8, rs, z[:, c:]) for w, (t8, rs), c in zip(wdevs, t8s, cols)], qd, sd, ldz)
    K.gemm_w8_segments([(w, None, rs, z2[:, c:]) for w, (_, rs), c in zip(w8s, t8s, cols)], qd, sd, ldz)
    assert np.array_equal(bits_of(z), ref.view(np.uint32))
    assert np.array_equal(bits_of(z2), ref.view(np.uint32))
    # the int32 accumulators and the BF16 output of the same products
    exact = np.concatenate([O.int_matmul(q, L.w8_reference()) for L in layers], 1)
    acc = torch.empty(M, ldz, dtype=torch.int32, device=DEV)
    K.gemm_tcq_segments([(w, t8, rs, acc[:, c:]) for w, (t8, rs), c in zip(wdevs, t8s, cols)], qd, None, ldz)
    assert np.array_equal(acc.cpu().numpy(), exact)
    yb = torch.empty(M, ldz, dtype=torch.bfloat16, device=DEV)
    K.gemm_w8_segments([(w, None, rs, yb[:, c:]) for w, (_, rs), c in zip(w8s, t8s, cols)], qd, sd, ldz)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), O.bf16_bits(ref))
    yb.fill_(float('nan'))
    K.gemm_tcq_segments([(w, t8, rs, yb[:, c:]) for w, (t8, rs), c in zip(wdevs, t8s, cols)], qd, sd, ldz)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), O.bf16_bits(ref))


@pytest.mark.parametrize('G,M', [(8, 1), (4, 9)])
def test_gemm_tcq_streaming_row_group_tables(G, M):
    """The streaming plan of the fused product (one token block, 2048 x 16384: 8192 chunks) with (G, 512, 2) row-group
    tables: every workgroup's rows read their group's table; FP32 bits equal the oracle's."""
    from yanlongvla_amd import kernels as K
    m, n = 2048, 16384
    L = O.random_layer(m, n, 70 + G, groups=G)
    d = dev_layer(L)
    t8, rs, _ = K.snap(d['tlut'], d['row_scale'])
    rng = np.random.default_rng(G + M)
    q = rng.integers(-127, 128, size=(M, n)).astype(np.int8)
    s = (rng.random(M) * 0.02 + 1e-3).astype(np.float32)
    ref = (O.int_matmul(q, L.w8_reference()).astype(np.float32) * s[:, None]) * L.rs[None, :]
    z = torch.full((M, m), float('nan'), device=DEV)
    K.gemm_tcq_segments([(K.repack(d['bits'], m, n), t8, rs, z)], T(q), T(s), m)
    assert np.array_equal(bits_of(z), ref.view(np.uint32))


@pytest.mark.parametrize('shapes,M,parts', [([(2048, 16384)], 1, 2), ([(2048, 2048)], 1, 2), ([(1024, 2048)], 50, 4),
                                            ([(1024, 4096)], 50, 4), ([(256, 512)], 3, 4), ([(2048, 1024), (256, 1024)], 17, 2),
                                            ([(2048, 16384)], 16, 4)])
def test_gemm_k_parts(shapes, M, parts):
    """K parts of the fused and the INT8-resident small-M products (streaming and workgroup plans): the int32 parts sum
    to the exact product; a part whose chunk range is empty (K = 512 in 4 parts: 2 chunks) writes zeros."""
    from yanlongvla_amd import kernels as K
    layers, dev, t8s, q, s, ldz, ref = _small_product_case(shapes, M, 7 * M + parts)
    n = layers[0].n
    qd, sd = T(q), T(s)
    exact = np.concatenate([O.int_matmul(q, L.w8_reference()) for L in layers], 1)
    wdevs = [K.repack(d['bits'], L.m, n) for L, d in zip(layers, dev)]
    w8s = []
    for L, d, (t8, _) in zip(layers, dev, t8s):
        w = torch.empty(L.m, n, dtype=torch.int8, device=DEV)
        K.decode(d['bits'], t8, w)
        w8s.append(w)
    cols = np.cumsum([0] + [L.m for L in layers])[:-1]
    nch = (n + 255) // 256
    per = (nch + parts - 1) // parts
    for resident in (False, True):
        acc = torch.full((parts, M, ldz), -12345, dtype=torch.int32, device=DEV)
        if resident:
            K.gemm_w8_segments([(w, None, rs, acc[0, :, c:]) for w, (_, rs), c in zip(w8s, t8s, cols)], qd, sd, ldz, parts)
        else:
            K.gemm_tcq_segments([(w, t8, rs, acc[0, :, c:]) for w, (t8, rs), c in zip(wdevs, t8s, cols)], qd, sd, ldz, parts)
        a = acc.cpu().numpy().astype(np.int64)
        assert np.array_equal(a.sum(0), exact), resident
        for p in range(parts):                                   # each part is the product over its own chunks
            k0, k1 = min(n, 256 * per * p), min(n, 256 * per * (p + 1))
            want = np.concatenate([O.int_matmul(q[:, k0:k1], L.w8_reference()[:, k0:k1]) if k1 > k0 else
                                   np.zeros((M, L.m), np.int64) for L in layers], 1)
            assert np.array_equal(a[p], want), (resident, p)
    with pytest.raises(ValueError):                              # K parts are int32 sums only
        K.gemm_tcq_segments([(wdevs[0], t8s[0][0], t8s[0][1], torch.empty(parts, M, ldz, device=DEV)[0])], qd, sd, ldz, parts)


@pytest.mark.parametrize('shapes,parts', [([(2048, 1024)], 1), ([(4112, 1024), (2048, 1024)], 1), ([(48, 80), (32, 80)], 1),
                                          ([(2048, 16384)], 1), ([(8192, 2048)] * 4, 1), ([(65536, 1024)], 1),
                                          ([(2048, 2560)], 1), ([(2048, 16384)], 2), ([(2048, 2048)], 2), ([(256, 512)], 4)])
def test_one_token_dot_products_bitexact(shapes, parts):
    """One-token products on dot-product instructions (DOT4): the workgroup plan with one and two tile rows per workgroup,
    the streaming plan at 16 / 4 / 1 waves per tile row, K parts on both plans, K = 80 (a partial chunk); fused decode
    and INT8-resident weights; FP32 / BF16 / int32 outputs, row-major and token-block activations. Every output equals
    the MFMA product's bits, and the FP32 / int32 ones the oracle's."""
    from yanlongvla_amd import kernels as K
    M = 1
    layers, dev, t8s, q, s, ldz, ref = _small_product_case(shapes, M, 5 * len(shapes) + parts)
    n = layers[0].n
    qd, sd = T(q), T(s)
    tb = K.token_blocks(M, n, DEV)
    qp = torch.zeros(16, n, dtype=torch.int8, device=DEV)
    qp[:M] = qd
    tb.copy_(qp.view(1, 16, n // 16, 16).permute(0, 2, 1, 3))
    exact = np.concatenate([O.int_matmul(q, L.w8_reference()) for L in layers], 1)
    wdevs = [K.repack(d['bits'], L.m, n) for L, d in zip(layers, dev)]
    w8s = []
    for L, d, (t8, _) in zip(layers, dev, t8s):
        w = torch.empty(L.m, n, dtype=torch.int8, device=DEV)
        K.decode(d['bits'], t8, w)
        w8s.append(w)
    cols = np.cumsum([0] + [L.m for L in layers])[:-1]
    dts = (torch.int32,) if parts > 1 else (torch.float32, torch.bfloat16, torch.int32)
    for resident, ws in ((False, wdevs), (True, w8s)):
        fn = K.gemm_w8_segments if resident else K.gemm_tcq_segments
        for dt in dts:
            for act in (qd, tb):
                out = {}
                for dot in (False, True):
                    z = torch.full((parts, M, ldz), -7, dtype=torch.int32, device=DEV).view(dt) if dt != torch.bfloat16 else \
                        torch.full((parts, M, ldz), float('nan'), dtype=dt, device=DEV)
                    fn([(w, None if resident else t8, rs, z[0, :, c:]) for w, (t8, rs), c in zip(ws, t8s, cols)], act,
                       None if (dt == torch.int32 and act is qd) else sd, ldz, parts, dot=dot)
                    out[dot] = z.view(torch.int16 if dt == torch.bfloat16 else torch.int32).cpu().numpy()
                case = (resident, dt, act is tb)
                assert np.array_equal(out[True], out[False]), case
                if dt == torch.int32:
                    assert np.array_equal(out[True].astype(np.int64).sum(0), exact), case
                elif dt == torch.float32:
                    assert np.array_equal(out[True][0].view(np.uint32), ref.view(np.uint32)), case
    with pytest.raises(ValueError):                                       # dot products take one token
        K.gemm_tcq_segments([(wdevs[0], t8s[0][0], t8s[0][1], torch.empty(2, ldz, device=DEV))], T(np.repeat(q, 2, 0)),
                            T(np.repeat(s, 2)), ldz, dot=True)


def test_one_token_dot_stage_split_middle():
    """The stage-split gated-MLP input (TCQ_Z_W128T) on dot-product instructions equals its MFMA form bit for bit."""
    from yanlongvla_amd import kernels as K
    N, n = 2048, 2048
    layers = [O.random_layer(N, n, 90 + i) for i in range(2)]
    dev = [dev_layer(L) for L in layers]
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, size=(1, n)).astype(np.int8)
    s = (rng.random(1) * 0.02 + 1e-3).astype(np.float32)
    segs = []
    for L, d in zip(layers, dev):
        t8, rs, _ = K.snap(d['tlut'], d['row_scale'])
        segs.append((K.repack(d['bits'], L.m, n), t8, rs))
    out = {}
    for dot in (False, True):
        zt = torch.full((2, 1, 128, N // 128), float('nan'), device=DEV)
        K.gemm_tcq_w128t([(w, t8, rs, zt[i]) for i, (w, t8, rs) in enumerate(segs)], T(q), T(s), dot=dot)
        out[dot] = zt.view(torch.int32).cpu().numpy()
    assert np.array_equal(out[True], out[False])
    assert not np.isnan(out[True].view(np.float32)).any()


def test_gemm_small_rejects_bad_sizes():
    from yanlongvla_amd import kernels as K, _lib
    L = O.random_layer(32, 64, 1)
    d = dev_layer(L)
    t8, rs, _ = K.snap(d['tlut'], d['row_scale'])
    q = torch.zeros(65, 64, dtype=torch.int8, device=DEV)
    s = torch.ones(65, device=DEV)
    z = torch.empty(65, 32, device=DEV)
    with pytest.raises(_lib.TcqError):
        K.gemm_tcq_segments([(K.repack(d['bits'], 32, 64), t8, rs, z)], q, s, 32)      # 65 tokens: more than the small-M product takes
    with pytest.raises(ValueError):
        K.gemm_tcq_segments([(K.repack(d['bits'], 32, 64), t8, rs, z)] * 5, q[:4], s[:4], 32)   # more segments than a launch takes


# ----------------------------------------------------------------------------------------------------------- W8A8 GEMM
@pytest.mark.parametrize('M,K,N', [(800, 2048, 16384), (50, 2048, 16384), (1, 2048, 16384), (33, 80, 48), (130, 1152, 260),
                                   (17, 16, 4),
                                   # 256-token tiles whose last tile holds 1 to 64 rows, K not a multiple of the 64-byte step
                                   (801, 256, 32768), (832, 64, 16384), (769, 208, 16384)])
def test_gemm_i8_bitexact(M, K, N):
    """INT32 accumulators equal the exact integer product; FP32 / BF16 epilogues equal (acc * sa) * sw bit for bit."""
    from yanlongvla_amd import kernels as Kk
    rng = np.random.default_rng(M + K + N)
    a = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    w = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    sa = (rng.random(M) * 0.03 + 1e-3).astype(np.float32)
    sw = (rng.random(N) * 1e-3 + 1e-5).astype(np.float32)
    ref = O.int_matmul(a, w)
    ad, wd = T(a), T(w)
    acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
    Kk.gemm_i8(ad, wd, acc)
    assert np.array_equal(acc.cpu().numpy(), ref)
    zf = (ref.astype(np.float32) * sa[:, None]) * sw[None, :]
    z = torch.empty(M, N, dtype=torch.float32, device=DEV)
    Kk.gemm_i8(ad, wd, z, T(sa), T(sw))
    assert np.array_equal(bits_of(z), zf.view(np.uint32))
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    Kk.gemm_i8(ad, wd, y, T(sa), T(sw))
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), O.bf16_bits(zf))


def test_w8a8_pipeline_matches_oracle():
    """C2 contract end to end: per-token INT8 of bf16 activations, per-channel INT8 of N(0, 0.02) weights, GEMM, BF16."""
    from yanlongvla_amd import kernels as Kk
    M, K, N = 50, 2048, 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g).bfloat16()
    wt = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    ref = O.w8a8_reference(x.float().numpy(), wt.float().numpy())
    qa = torch.empty(M, K, dtype=torch.int8, device=DEV)
    sa = torch.empty(M, device=DEV)
    Kk.quantize_rows(x.to(DEV), qa, sa)
    qw = torch.empty(N, K, dtype=torch.int8, device=DEV)
    sw = torch.empty(N, device=DEV)
    Kk.quantize_rows(wt.to(DEV), qw, sw)
    assert np.array_equal(qa.cpu().numpy(), ref['qa']) and np.array_equal(qw.cpu().numpy(), ref['qw'])
    assert np.array_equal(bits_of(sa), ref['sa'].view(np.uint32)) and np.array_equal(bits_of(sw), ref['sw'].view(np.uint32))
    acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
    Kk.gemm_i8(qa, qw, acc)
    assert np.array_equal(acc.cpu().numpy(), ref['acc'])
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    Kk.gemm_i8(qa, qw, y, sa, sw)
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), ref['y'])
