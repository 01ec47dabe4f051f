"""The W2 float path (BF16 rotated activations, the INT8 table values as weights, FP32 sums) through the C ABI, with the
reference's own arguments (deploy/tcq_kernels/kernels.py:677-696) and call sequence (Group.run_float, modules.py:117-144):

  pre_h        bf16(fwht(x * su)) into h (M, K) and hT (K, ldh), bit for bit against the oracle's fwht + BF16 rounding
  gemmf_*      the reference-shaped products (hT activations, stored words with bounds / resident INT8 weights) and the
               segment forms the module layer uses: the FP32 sums within 1e-6 of the FP64 product of the same operands, the
               fused decode and the resident weights bit-identical to each other, and the layer outputs of the reference's
               run_float sequence within 2e-3 of the oracle's w2_linear (the layer definition, FP64 sums)
  mid2_available  the widths tcq_mid2 takes."""
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


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def group_layers(shapes, seed):
    """Layers of one group (shared input signs) as device Layers and oracle twins."""
    from yanlongvla_amd import tcq_format as F
    ols = [O.random_layer(m, shapes[0][1], seed + i, per_layer_scale=False) for i, (m, _) in enumerate(shapes)]
    for ol in ols[1:]:
        ol.su = ols[0].su
    devs = [F.Layer(f'l{i}', dict(bits=T(ol.bits), tlut=T(ol.tlut), row_scale=T(ol.row_scale), su=T(ol.su), sv=T(ol.sv)),
                    device=DEV) for i, ol in enumerate(ols)]
    return devs, ols


@pytest.mark.parametrize('M,K', [(1, 1024), (10, 2048), (50, 4096), (7, 4304), (3, 16384), (64, 256)])
@pytest.mark.parametrize('xdt', [torch.bfloat16, torch.float32])
def test_pre_h_bitexact(M, K, xdt):
    from yanlongvla_amd import kernels as Kn
    rng = np.random.default_rng(M * K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    su = np.where(rng.integers(0, 2, K) > 0, 1, -1).astype(np.int8)
    xd = T(x).to(xdt)
    want = O.bf16_bits(O.fwht(xd.float().cpu().numpy() * su.astype(np.float32)))
    ldh = M + 3
    h = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    hT = torch.zeros(K, ldh, dtype=torch.bfloat16, device=DEV)
    Kn.pre_h(xd, T(su), h=h, hT=hT)
    assert np.array_equal(bits16(h), want)
    got = bits16(hT)
    assert np.array_equal(got[:, :M].T, want) and (got[:, M:] == 0).all()
    h2 = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    Kn.pre_h(xd, T(su), h=h2)                                  # row-major only: the rotation engines
    assert np.array_equal(bits16(h2), want)


def product_fp64(h_bits, w8, rs):
    return (O.bf16_to_f32(h_bits).astype(np.float64) @ w8.astype(np.float64).T) * rs.astype(np.float64)[None, :]


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize('M', [1, 10, 50, 64])
@pytest.mark.parametrize('shapes', [[(2048, 1024), (256, 1024), (256, 1024)], [(4096, 1024), (4096, 1024)],
                                    [(1024, 4096)], [(512, 4304)]])
def test_reference_run_float_sequence(shapes, M):
    """Group.run_float's expert branch (modules.py:131-144) on the reference-shaped helpers: hT = pre_h(x, su, hT=hT);
    z = gemmf_w8(W, hT, rs, z) or gemmf_tcq(bits, t8, hT, rs, z, K, bounds) over the concatenated layers; post per layer."""
    from yanlongvla_amd import kernels as Kn
    devs, ols = group_layers(shapes, 40 + M)
    K = shapes[0][1]
    N = [m for m, _ in shapes]
    col0 = [sum(N[:i]) for i in range(len(N))]
    Ntot = sum(N)
    bits = torch.cat([L.bits for L in devs]).contiguous()
    t8 = torch.cat([L.t8.reshape(-1) for L in devs]).contiguous()
    rs = torch.cat([L.rs for L in devs]).contiguous()
    bounds = [c // 16 for c in col0[1:]] + [1 << 30] * (3 - len(devs))
    W = torch.empty(Ntot, K, dtype=torch.int8, device=DEV)
    for L, c in zip(devs, col0):
        Kn.decode(L.bits, L.t8, W[c:c + L.m])
    x = T(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32)).bfloat16()
    hT = torch.empty(K, M, dtype=torch.bfloat16, device=DEV)
    Kn.pre_h(x, devs[0].su, hT=hT)
    z_w8 = torch.empty(M, Ntot, device=DEV)
    Kn.gemmf_w8(W, hT, rs, z_w8)
    z_tcq = torch.empty(M, Ntot, device=DEV)
    Kn.gemmf_tcq(bits, t8, hT, rs, z_tcq, K, bounds)
    assert torch.equal(z_w8, z_tcq)                            # same values, same MFMA order
    w8 = np.concatenate([ol.w8_reference() for ol in ols])
    want = product_fp64(bits16(hT).T, w8, rs.cpu().numpy())
    assert rel(z_w8.cpu().numpy(), want) < 1e-6
    xs = x.float().cpu().numpy()
    for L, ol, c in zip(devs, ols, col0):
        y = torch.empty(M, L.m, dtype=torch.bfloat16, device=DEV)
        Kn.post(z_w8, None, None, L.sv, None, y, col0=c)
        ref = O.bf16_to_f32(O.w2_linear(xs, ol, small=True))
        assert rel(O.bf16_to_f32(bits16(y)), ref) < 2e-3


@pytest.mark.parametrize('M', [1, 16, 33, 64, 100, 200])
@pytest.mark.parametrize('odt', [torch.float32, torch.bfloat16])
def test_gemmf_segments(M, odt):
    """The segment forms on row-major activations: repacked words (fused decode) and resident INT8 weights give the same
    bits; FP32 out = sum * rs within 1e-6 of FP64; BF16 out = the unscaled sum rounded once (within one BF16 rounding of
    the FP64 sum). M > 64 runs in groups of 64 tokens (grid.z)."""
    from yanlongvla_amd import kernels as Kn
    shapes = [(2048, 2048), (256, 2048), (256, 2048)]
    devs, ols = group_layers(shapes, 70 + M)
    K, Ntot = 2048, sum(m for m, _ in shapes)
    x = T(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32)).bfloat16()
    h = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    Kn.pre_h(x, devs[0].su, h=h)
    col0 = [0, 2048, 2304]
    outs = {}
    for resident in (False, True):
        out = torch.full((M, Ntot), float('nan'), dtype=odt, device=DEV)
        segs = [((L.w8_reference() if resident else L.words()), None if resident else L.t8, L.rs, out[:, c:])
                for L, c in zip(devs, col0)]
        Kn.gemmf_segments(segs, h, Ntot, resident=resident)
        outs[resident] = out
    assert torch.equal(outs[False], outs[True])
    w8 = np.concatenate([ol.w8_reference() for ol in ols])
    if odt == torch.float32:
        want = product_fp64(bits16(h), w8, np.concatenate([ol.rs for ol in ols]))
        assert rel(outs[False].cpu().numpy(), want) < 1e-6
    else:
        want = product_fp64(bits16(h), w8, np.ones(Ntot, np.float32))
        got = outs[False].float().cpu().numpy()
        assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6 * np.abs(want).max())


def test_mid2_available():
    from yanlongvla_amd import kernels as Kn
    assert Kn.mid2_available(4096) and Kn.mid2_available(16384) and Kn.mid2_available(4304)
    assert not Kn.mid2_available(16400) and not Kn.mid2_available(24) and not Kn.mid2_available(0)
