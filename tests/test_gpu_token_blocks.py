"""GPU tests of the token-block activation layout: every quantizing entry point writes through its q4 output (ldq =
LDQ_TOKEN_BLOCKS) exactly the bytes of its row-major q output rearranged, and the small-M products give the same bits from
token blocks as from row-major activations. Engine paths covered: rows of 1024 / 2048 / 4096 (16 values per thread),
8192 (register path of the fused norm kernel), 1152 (LDS engine)."""
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
    return T(np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8))


def bf16(rng, *shape):
    return T(rng.standard_normal(shape).astype(np.float32)).bfloat16()


def outs(M, K):
    from yanlongvla_amd import kernels as K_
    return (torch.empty(M, K, dtype=torch.int8, device=DEV), K_.token_blocks(M, K, DEV), torch.empty(M, device=DEV),
            torch.empty(M, device=DEV))


def same(q, tb, s1, s2, M):
    from yanlongvla_amd import kernels as K_
    assert torch.equal(K_.rows_of_token_blocks(tb, M), q)
    assert torch.equal(s1, s2)


def test_token_block_view_is_the_documented_layout():
    """rows_of_token_blocks against the byte formula of the layout, on the CPU side of a device tensor."""
    from yanlongvla_amd import kernels as K_
    M, K = 20, 48
    tb = K_.token_blocks(M, K, DEV)
    flat = torch.arange(tb.numel(), dtype=torch.int32).remainder(251).to(torch.int8)
    tb.view(-1).copy_(flat.to(DEV))
    rows = K_.rows_of_token_blocks(tb, M).cpu().numpy()
    raw = tb.view(-1).cpu().numpy()
    for t in range(M):
        for k in range(K):
            assert rows[t, k] == raw[((t // 16 * (K // 16) + k // 16) * 16 + t % 16) * 16 + k % 16]


@pytest.mark.parametrize('M,K', [(1, 1024), (17, 2048), (50, 4096), (5, 1152)])
def test_pre_and_norm_pre(M, K):
    from yanlongvla_amd import kernels as K_
    rng = np.random.default_rng(M + K)
    x, su, w = bf16(rng, M, K), signs(rng, K), bf16(rng, K)
    q, tb, s1, s2 = outs(M, K)
    K_.pre(x, su, q=q, scale=s1)
    K_.pre(x, su, q4=tb, scale=s2)
    same(q, tb, s1, s2, M)
    K_.norm_pre(x, w, 1e-6, su, q=q, scale=s1)
    K_.norm_pre(x, w, 1e-6, su, q4=tb, scale=s2)
    same(q, tb, s1, s2, M)


@pytest.mark.parametrize('M,N', [(1, 1024), (17, 2048), (50, 4096), (3, 8192), (5, 1152)])
def test_post_add_norm_pre(M, N):
    from yanlongvla_amd import kernels as K_
    rng = np.random.default_rng(M * 3 + N)
    acc = T(rng.standard_normal((M, N)).astype(np.float32))
    x, w, sv, su = bf16(rng, M, N), bf16(rng, N), signs(rng, N), signs(rng, N)
    q, tb, s1, s2 = outs(M, N)
    x1, x2 = torch.empty_like(x), torch.empty_like(x)
    K_.post_add_norm_pre(acc, None, None, sv, None, x, x1, w, 1e-6, su, q=q, scale=s1)
    K_.post_add_norm_pre(acc, None, None, sv, None, x, x2, w, 1e-6, su, q4=tb, scale=s2)
    same(q, tb, s1, s2, M)
    assert torch.equal(x1, x2)


@pytest.mark.parametrize('M,N', [(1, 4096), (50, 4096), (17, 1024), (3, 16384), (4, 1152)])
def test_middles_and_pre2(M, N):
    from yanlongvla_amd import kernels as K_
    rng = np.random.default_rng(M * 5 + N)
    acc = T(rng.standard_normal((M, 2 * N)).astype(np.float32))
    sv, su = signs(rng, 2 * N), signs(rng, N)
    q, tb, s1, s2 = outs(M, N)
    K_.mid2(acc, None, None, sv, su, q=q, scale=s1)
    K_.mid2(acc, None, None, sv, su, q4=tb, scale=s2)
    same(q, tb, s1, s2, M)
    a1 = T(rng.standard_normal((M, N)).astype(np.float32))
    K_.mid1(a1, None, None, sv[:N].contiguous(), None, su, q=q, scale=s1)
    K_.mid1(a1, None, None, sv[:N].contiguous(), None, su, q4=tb, scale=s2)
    same(q, tb, s1, s2, M)
    g, u = bf16(rng, M, N), bf16(rng, M, N)
    K_.pre2(g, u, su, q=q, scale=s1)
    K_.pre2(g, u, su, q4=tb, scale=s2)
    same(q, tb, s1, s2, M)


@pytest.mark.parametrize('M,P,H', [(50, 800, 8), (1, 832, 8), (17, 100, 4), (3, 63, 2)])
def test_attention_prologue(M, P, H):
    from yanlongvla_amd import kernels as K_
    rng = np.random.default_rng(M + P)
    q = bf16(rng, M, H * 256)
    kc, vc, kn, vn = bf16(rng, P, 256), bf16(rng, P, 256), bf16(rng, M, 256), bf16(rng, M, 256)
    su = signs(rng, H * 256)
    q8, tb, s1, s2 = outs(M, H * 256)
    K_.attend(q, kc, vc, kn, vn, H, None, su=su, q8=q8, scale=s1)
    K_.attend(q, kc, vc, kn, vn, H, None, su=su, q4=tb, scale=s2)
    same(q8, tb, s1, s2, M)


@pytest.mark.parametrize('M', [1, 17, 50, 64])
def test_small_products_from_token_blocks(M):
    """gemm_tcq (fused decode) and gemm_w8 (resident INT8) over three segments: FP32 and int32 outputs equal bit for bit."""
    from yanlongvla_amd import kernels as K_
    rng = np.random.default_rng(M)
    Kd = 1024
    layers = [O.random_layer(m, Kd, 100 + i) for i, m in enumerate((256, 64, 96))]
    q = T(rng.integers(-127, 128, size=(M, Kd)).astype(np.int8))
    s = T((rng.random(M) * 1e-2 + 1e-3).astype(np.float32))
    tb = K_.token_blocks(M, Kd, DEV)
    B, G = tb.shape[0], tb.shape[1]
    qp = torch.zeros(B * 16, Kd, dtype=torch.int8, device=DEV)
    qp[:M] = q
    tb.copy_(qp.view(B, 16, G, 16).permute(0, 2, 1, 3))                                # rows -> token blocks
    assert torch.equal(K_.rows_of_token_blocks(tb, M), q)
    cols = [int(c) for c in np.cumsum([0] + [L.m for L in layers])[:-1]]
    ldz = sum(L.m for L in layers)
    segs_t, segs_w = [], []
    for L in layers:
        t8, rs, _ = K_.snap(T(L.tlut.view(np.int16)), T(L.row_scale.view(np.int16)))
        w8 = torch.empty(L.m, Kd, dtype=torch.int8, device=DEV)
        K_.decode(T(L.bits), t8, w8)
        segs_t.append((K_.repack(T(L.bits), L.m, Kd), t8, rs))
        segs_w.append((w8, None, rs))
    for segs, fn in ((segs_t, K_.gemm_tcq_segments), (segs_w, K_.gemm_w8_segments)):
        for dt in (torch.float32, torch.int32):
            z1 = torch.empty(M, ldz, dtype=dt, device=DEV)
            z2 = torch.empty_like(z1)
            fn([(a, b, r, z1[:, c:]) for (a, b, r), c in zip(segs, cols)], q, s if dt == torch.float32 else None, ldz)
            fn([(a, b, r, z2[:, c:]) for (a, b, r), c in zip(segs, cols)], tb, s, ldz)     # token blocks: M = s.numel()
            assert torch.equal(z1.view(torch.int32), z2.view(torch.int32))


def test_token_block_argument_errors():
    """K % 16 != 0 and a misaligned token-block buffer are refused before any launch."""
    from yanlongvla_amd import _lib
    lib = _lib.lib()
    x = torch.zeros(2, 40, dtype=torch.bfloat16, device=DEV)
    su = torch.ones(40, dtype=torch.int8, device=DEV)
    tb = torch.zeros(4096, dtype=torch.int8, device=DEV)
    s = torch.zeros(2, device=DEV)
    P = lambda t, off=0: t.data_ptr() + off
    assert lib.tcq_pre(P(x), 1, P(su), None, P(tb), -16, P(s), 2, 40, None) == -2          # K = 40: not a multiple of 16
    x2 = torch.zeros(2, 64, dtype=torch.bfloat16, device=DEV)
    su2 = torch.ones(64, dtype=torch.int8, device=DEV)
    assert lib.tcq_pre(P(x2), 1, P(su2), None, P(tb, 4), -16, P(s), 2, 64, None) == -5     # token blocks off 16 bytes
    assert lib.tcq_pre(P(x2), 1, P(su2), None, P(tb), 1, P(s), 2, 64, None) == -1           # word layout with ldq < M
