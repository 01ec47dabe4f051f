"""GPU parity of the fused MLP middles (gated GeGLU middle, plain GELU middle, split second half) against the oracle:
INT8 activations and per-token scales bit-exact, for int32 / FP32 / BF16 accumulators and Walsh widths made of one or
several power-of-two blocks."""
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


def signs(rng, n):
    return np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8)


def lut_np():
    from yanlongvla_amd import kernels as K
    return K.gelu_table(DEV).view(torch.int16).cpu().numpy().view(np.uint16)


def accumulators(rng, M, width, kind):
    """Random accumulators of one kind and the scaled FP32 rows the kernels see: int32 -> (float(a) * s) * rs,
    BF16 -> bf16(a) * rs, FP32 -> a."""
    if kind == 'i32':
        acc = rng.integers(-2 ** 18, 2 ** 18, size=(M, width)).astype(np.int32)
        s = (rng.random(M) * 1e-3 + 1e-4).astype(np.float32)
        rs = (rng.random(width) * 1e-2 + 1e-3).astype(np.float32)
        z = (acc.astype(np.float32) * s[:, None]) * rs[None, :]
        return T(acc), T(s), T(rs), z
    if kind == 'bf16':
        a = O.bf16_bits(rng.standard_normal((M, width)).astype(np.float32))
        rs = (rng.random(width) + 0.5).astype(np.float32)
        z = O.bf16_to_f32(a) * rs[None, :]
        return T(a.view(np.int16)).view(torch.bfloat16), None, T(rs), z
    acc = rng.standard_normal((M, width)).astype(np.float32)
    return T(acc), None, None, acc


@pytest.mark.parametrize('kind', ['i32', 'f32', 'bf16'])
@pytest.mark.parametrize("M,N", [(1, 4096), (50, 4096), (3, 16384), (1, 16384), (7, 1152), (2, 48), (4, 1024), (2, 2048),
                                 (3, 8192), (70, 8192)])
def test_mid2_bitexact(kind, M, N):
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(M * 7 + N)
    acc, s, rs, z = accumulators(rng, M, 2 * N, kind)
    sv, su = signs(rng, 2 * N), signs(rng, N)
    q = torch.empty(M, N, dtype=torch.int8, device=DEV)
    q4 = torch.empty(N // 4, M, dtype=torch.int32, device=DEV)
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid2(acc, s, rs, T(sv), T(su), q=q, q4=q4, scale=sc)
    lut = lut_np()
    qr, sr, _, _ = O.mlp_middle(z[:, :N], z[:, N:], sv[:N], sv[N:], su, gelu=lambda b: lut[b])
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(sc.cpu().numpy(), sr[:, 0])
    assert np.array_equal(q4.cpu().numpy(), O.q4_layout(qr))


@pytest.mark.parametrize('N', [4096, 16384])
def test_mid2_gelu_inputs_of_every_magnitude(N):
    """Rows scaled from 2^-40 to 2^20 (and a zero row): gate values below, inside and above the exponent window whose GELU
    results the kernel keeps in LDS, so both the LDS copy and the global table are read; bit-exact against the oracle."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(N + 5)
    M = 25
    z = rng.standard_normal((M, 2 * N)).astype(np.float32)
    z *= np.exp2(np.linspace(-40, 20, M)).astype(np.float32)[:, None]
    z[M // 2] = 0
    sv, su = signs(rng, 2 * N), signs(rng, N)
    q = torch.empty(M, N, dtype=torch.int8, device=DEV)
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid2(T(z), None, None, T(sv), T(su), q=q, scale=sc)
    lut = lut_np()
    qr, sr, _, _ = O.mlp_middle(z[:, :N], z[:, N:], sv[:N], sv[N:], su, gelu=lambda b: lut[b])
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(sc.cpu().numpy(), sr[:, 0])


@pytest.mark.parametrize('N', [1024, 4096])
def test_mid2_strided_accumulator(N):
    """Gate | up columns inside a wider accumulator row (lda > 2N), as when more layers share the product."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(11 + N)
    M, lda = 5, 2 * N + 256
    full = rng.integers(-2 ** 18, 2 ** 18, size=(M, lda)).astype(np.int32)
    s = (rng.random(M) * 1e-3 + 1e-4).astype(np.float32)
    rs = (rng.random(2 * N) * 1e-2).astype(np.float32)
    sv, su = signs(rng, 2 * N), signs(rng, N)
    q = torch.empty(M, N, dtype=torch.int8, device=DEV)
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid2(T(full), T(s), T(rs), T(sv), T(su), q=q, scale=sc)
    z = (full[:, :2 * N].astype(np.float32) * s[:, None]) * rs[None, :]
    lut = lut_np()
    qr, sr, _, _ = O.mlp_middle(z[:, :N], z[:, N:], sv[:N], sv[N:], su, gelu=lambda b: lut[b])
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(sc.cpu().numpy(), sr[:, 0])


@pytest.mark.parametrize('kind', ['i32', 'f32', 'bf16'])
@pytest.mark.parametrize("M,N,with_bias", [(1, 4304, True), (50, 4096, False), (10, 1152, True), (4, 48, True)])
def test_mid1_bitexact(kind, M, N, with_bias):
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(M * 13 + N)
    acc, s, rs, z = accumulators(rng, M, N, kind)
    sv, su = signs(rng, N), signs(rng, N)
    bias = (rng.standard_normal(N) * 0.2).astype(np.float32) if with_bias else None
    q = torch.empty(M, N, dtype=torch.int8, device=DEV)
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid1(acc, s, rs, T(sv), None if bias is None else T(bias), T(su), q=q, scale=sc)
    lut = lut_np()
    qr, sr, _ = O.plain_middle(z, sv, bias, su, gelu=lambda b: lut[b])
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(sc.cpu().numpy(), sr[:, 0])


@pytest.mark.parametrize('M,K', [(1, 16384), (50, 4096), (9, 1152), (3, 8)])
def test_pre2_bitexact(M, K):
    from yanlongvla_amd import kernels as Kn
    rng = np.random.default_rng(M + K)
    g = O.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    u = O.bf16_bits(rng.standard_normal((M, K)).astype(np.float32) * 3)
    su = signs(rng, K)
    q = torch.empty(M, K, dtype=torch.int8, device=DEV)
    q4 = torch.empty(K // 4, M + 3, dtype=torch.int32, device=DEV)          # ldq > M
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    Kn.pre2(T(g.view(np.int16)).view(torch.bfloat16), T(u.view(np.int16)).view(torch.bfloat16), T(su), q=q, q4=q4, scale=sc)
    qr, sr = O.pre2(g, u, su)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(sc.cpu().numpy(), sr[:, 0])
    assert np.array_equal(q4.cpu().numpy()[:, :M], O.q4_layout(qr))


def test_mid2_equals_split_middle():
    """mid2 == postg(gate with GELU, up) followed by pre2: the fused kernel changes no rounding point."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(5)
    M, N = 50, 4096
    acc, s, rs, _ = accumulators(rng, M, 2 * N, 'i32')
    sv, su = T(signs(rng, 2 * N)), T(signs(rng, N))
    q1 = torch.empty(M, N, dtype=torch.int8, device=DEV)
    s1 = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid2(acc, s, rs, sv, su, q=q1, scale=s1)
    g = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    u = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    desc = K.post_segments([(acc, 0, rs[:N], sv[:N], None, g, True), (acc, N, rs[N:], sv[N:], None, u, False)], DEV)
    K.post_batched(desc, 2, torch.int32, torch.bfloat16, s, M, N, gelu_lut=K.gelu_table(DEV))
    q2 = torch.empty(M, N, dtype=torch.int8, device=DEV)
    s2 = torch.empty(M, dtype=torch.float32, device=DEV)
    K.pre2(g, u, su, q=q2, scale=s2)
    assert torch.equal(q1, q2) and torch.equal(s1, s2)


@pytest.mark.parametrize('kind', ['i32', 'f32', 'bf16'])
@pytest.mark.parametrize('M,N', [(300, 4096), (800, 16384), (257, 1024), (400, 8192), (260, 2048)])
def test_mid2_many_rows_bitexact(kind, M, N):
    """More than 256 token rows: the one-row-per-transform branch of tcq_mid2 (the 800-token backbone prefill middle),
    bit-exact against the oracle for q, the (N/4, M) word layout and the token-block layout of q4."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(M * 3 + N + len(kind))
    acc, s, rs, z = accumulators(rng, M, 2 * N, kind)
    sv, su = signs(rng, 2 * N), signs(rng, N)
    q = torch.empty(M, N, dtype=torch.int8, device=DEV)
    q4 = torch.empty(N // 4, M, dtype=torch.int32, device=DEV)
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid2(acc, s, rs, T(sv), T(su), q=q, q4=q4, scale=sc)
    qb = K.token_blocks(M, N, DEV)
    sc2 = torch.empty(M, dtype=torch.float32, device=DEV)
    K.mid2(acc, s, rs, T(sv), T(su), q4=qb, scale=sc2)
    lut = lut_np()
    qr, sr, _, _ = O.mlp_middle(z[:, :N], z[:, N:], sv[:N], sv[N:], su, gelu=lambda b: lut[b])
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(sc.cpu().numpy(), sr[:, 0]) and np.array_equal(sc2.cpu().numpy(), sr[:, 0])
    assert np.array_equal(q4.cpu().numpy(), O.q4_layout(qr))
    assert np.array_equal(K.rows_of_token_blocks(qb, M).cpu().numpy(), qr)


@pytest.mark.parametrize('M', [1, 3, 16])
def test_spread_middle_equals_mid2_and_oracle(M):
    """The 16384-wide GeGLU middle of few tokens spread over many CUs: the gate/up product with the first seven Walsh
    stages in its epilogue (gemm_tcq_w128t), glu_split, then pre with the down projection's signs. Pinned three ways:
    the stage-split product's output equals the product's FP32 z after Walsh stages h = 1 .. 64 within 128-row blocks
    (computed on the host in the oracle's butterfly order), block-transposed, bit for bit; the INT8 rows and scales equal
    the one-launch mid2's bit for bit; and both equal the oracle's mlp_middle."""
    from yanlongvla_amd import kernels as K
    from yanlongvla_amd import tcq_format as F
    rng = np.random.default_rng(600 + M)
    n, N = 2048, 16384
    ols = [O.random_layer(N, n, 700 + M + i, per_layer_scale=False) for i in range(2)]
    ols[1].su = ols[0].su
    devs = [F.Layer(f'l{i}', dict(bits=T(ol.bits), tlut=T(ol.tlut), row_scale=T(ol.row_scale), su=T(ol.su), sv=T(ol.sv)),
                    device=DEV) for i, ol in enumerate(ols)]
    x = T(rng.standard_normal((M, n)).astype(np.float32)).bfloat16()
    tb, s = K.token_blocks(M, n, DEV), torch.empty(M, device=DEV)
    K.pre(x, devs[0].su, q4=tb, scale=s)
    z = torch.empty(M, 2 * N, device=DEV)
    K.gemm_tcq_segments([(L.words(), L.t8, L.rs, z[:, i * N:]) for i, L in enumerate(devs)], tb, s, 2 * N)
    zt = torch.empty(2, M, 128, 128, device=DEV)
    K.gemm_tcq_w128t([(L.words(), L.t8, L.rs, zt[i]) for i, L in enumerate(devs)], tb, s)
    # the first seven stages, on the host: (M, 2, 128 blocks, 128) -> butterflies h = 1 .. 64 within each block
    blocks = z.cpu().numpy().reshape(M, 2, 128, 128)
    h = 1
    while h < 128:
        v = blocks.reshape(M, 2, 128, 128 // (2 * h), 2, h)
        a, b = v[..., 0, :], v[..., 1, :]
        blocks = np.stack((a + b, a - b), axis=-2).reshape(M, 2, 128, 128)
        h *= 2
    want_zt = blocks.transpose(1, 0, 3, 2)                         # (2, M, offset, block)
    assert np.array_equal(zt.cpu().numpy().view(np.uint32), np.ascontiguousarray(want_zt).view(np.uint32))
    sv = torch.cat([L.sv for L in devs]).contiguous()
    su = T(signs(rng, N))
    lut = K.gelu_table(DEV)
    q1, s1 = K.token_blocks(M, N, DEV), torch.empty(M, device=DEV)
    K.mid2(z, None, None, sv, su, q4=q1, scale=s1, gelu_lut=lut)
    p = K.glu_split(zt, sv, lut, torch.empty(M, N, dtype=torch.bfloat16, device=DEV))
    q2, s2 = K.token_blocks(M, N, DEV), torch.empty(M, device=DEV)
    K.pre(p, su, q4=q2, scale=s2)
    assert torch.equal(K.rows_of_token_blocks(q1, M), K.rows_of_token_blocks(q2, M)) and torch.equal(s1, s2)
    zz = z.cpu().numpy()
    lut_h = lut.view(torch.int16).cpu().numpy().view(np.uint16)
    qr, sr, _, _ = O.mlp_middle(zz[:, :N], zz[:, N:], sv.cpu().numpy()[:N], sv.cpu().numpy()[N:], su.cpu().numpy(),
                                gelu=lambda b: lut_h[b])
    assert np.array_equal(K.rows_of_token_blocks(q2, M).cpu().numpy(), qr) and np.array_equal(s2.cpu().numpy(), sr[:, 0])
