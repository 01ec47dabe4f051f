"""GPU tests of the few-row kernels on the no-transpose Walsh engine (rows held 4 or 8 values per thread by 4 or 8 waves,
one LDS exchange per transform): below 65 rows, tcq_post_add_norm_pre (1024 / 2048 wide, with the norm), tcq_mid2 (1024 ..
4096 wide) and tcq_post_group (segments of 256 / 2048) take them; from 65 rows on, the register + transpose kernels. Every
row is computed on its own, so the first rows of a 65-row call and a 5-row call on the same inputs must hold the same bits:
the two engines run the same butterflies in the same stage order, the same sum-of-squares tree and the same roundings. The
many-row kernels are pinned against the oracle in test_gpu_norms.py, test_gpu_mlp.py and test_gpu_kernels.py."""
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = 'cuda'
FEW, MANY = 5, 65


@pytest.fixture(scope='module', autouse=True)
def _lib():
    from yanlongvla_amd import _lib
    _lib.lib()
    torch.cuda.init()


def signs(g, n):
    return (torch.randint(0, 2, (n,), generator=g, device=DEV) * 2 - 1).to(torch.int8)


def bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32 if t.element_size() == 4 else torch.int8).cpu()


def acc_of(dtype, shape, g):
    if dtype == torch.int32:
        return torch.randint(-(1 << 20), 1 << 20, shape, generator=g, device=DEV, dtype=torch.int32)
    a = torch.randn(shape, generator=g, device=DEV) * 3
    return a.bfloat16() if dtype == torch.bfloat16 else a


@pytest.mark.parametrize('N', [1024, 2048])
@pytest.mark.parametrize('adt,parts', [(torch.int32, 1), (torch.int32, 2), (torch.float32, 1), (torch.bfloat16, 1)])
def test_post_add_norm_pre_few_rows_equal_many(N, adt, parts):
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=DEV).manual_seed(N + parts + 7 * (adt == torch.float32))
    acc = acc_of(adt, (parts, MANY, N) if parts > 1 else (MANY, N), g)
    s = torch.rand(MANY, generator=g, device=DEV) * 1e-3 + 1e-4
    rs = torch.rand(N, generator=g, device=DEV) * 1e-3
    sv, su = signs(g, N), signs(g, N)
    x = torch.randn(MANY, N, generator=g, device=DEV).bfloat16()
    w = (torch.randn(N, generator=g, device=DEV) * 0.1).bfloat16()
    out = {}
    for M in (MANY, FEW):
        a = acc[:, :M].contiguous() if parts > 1 else acc[:M].contiguous()
        xo = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        q = torch.empty(M, N, dtype=torch.int8, device=DEV)
        q4 = K.token_blocks(M, N, DEV)
        sc = torch.empty(M, device=DEV)
        K.post_add_norm_pre(a, s[:M] if adt == torch.int32 else None, rs if adt != torch.float32 else None, sv, None, x[:M].contiguous(),
                            xo, w, 1e-6, su, q=q, scale=sc)
        K.post_add_norm_pre(a, s[:M] if adt == torch.int32 else None, rs if adt != torch.float32 else None, sv, None, x[:M].contiguous(),
                            torch.empty_like(xo), w, 1e-6, su, q4=q4, scale=torch.empty_like(sc))
        out[M] = (xo, q, sc, K.rows_of_token_blocks(q4, M))
    torch.cuda.synchronize()
    for a, b in zip(out[FEW], out[MANY]):
        assert torch.equal(bits(a), bits(b[:FEW]))
    assert torch.equal(out[FEW][1].cpu(), out[FEW][3].cpu())        # q and the token-block copy hold the same row


@pytest.mark.parametrize('N', [1024, 2048, 4096])
@pytest.mark.parametrize('adt', [torch.int32, torch.float32, torch.bfloat16])
def test_mid2_few_rows_equal_many(N, adt):
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=DEV).manual_seed(N + 3 * (adt == torch.int32))
    acc = acc_of(adt, (MANY, 2 * N), g)
    if adt == torch.float32:
        acc = acc * 0.05
    s = torch.rand(MANY, generator=g, device=DEV) * 1e-4 + 1e-5
    rs = torch.rand(2 * N, generator=g, device=DEV) * 1e-2
    sv, su = signs(g, 2 * N), signs(g, N)
    out = {}
    for M in (MANY, FEW):
        q = torch.empty(M, N, dtype=torch.int8, device=DEV)
        sc = torch.empty(M, device=DEV)
        K.mid2(acc[:M].contiguous(), s[:M] if adt == torch.int32 else None, rs if adt != torch.float32 else None, sv, su, q=q, scale=sc)
        out[M] = (q, sc)
    torch.cuda.synchronize()
    for a, b in zip(out[FEW], out[MANY]):
        assert torch.equal(bits(a), bits(b[:FEW]))


@pytest.mark.parametrize('ydt', [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize('adt', [torch.int32, torch.float32, torch.bfloat16])
def test_post_group_few_rows_equal_many(ydt, adt):
    """q / k / v shaped groups (2048, 256, 256) with a bias on one segment and GELU on another (BF16 out only)."""
    from yanlongvla_amd import kernels as K
    g = torch.Generator(device=DEV).manual_seed(11 + 5 * (ydt == torch.float32))
    widths = [2048, 256, 256]
    Nt = sum(widths)
    acc = acc_of(adt, (MANY, Nt), g)
    s = torch.rand(MANY, generator=g, device=DEV) * 1e-3 + 1e-4
    rs = torch.rand(Nt, generator=g, device=DEV) * 1e-3
    sv = signs(g, Nt)
    bias = torch.randn(256, generator=g, device=DEV)
    lut = K.gelu_table(DEV) if ydt == torch.bfloat16 else None
    out = {}
    for M in (MANY, FEW):
        a = acc[:M].contiguous()
        ys, segs, c0 = [], [], 0
        for i, n in enumerate(widths):
            y = torch.empty(M, n, dtype=ydt, device=DEV)
            segs.append((a, c0, rs[c0:c0 + n] if adt != torch.float32 else None, sv[c0:c0 + n], bias if i == 1 else None, y,
                         lut is not None and i == 2))
            ys.append(y)
            c0 += n
        K.post_group(segs, adt, ydt, s[:M] if adt == torch.int32 else None, M, gelu_lut=lut)
        out[M] = ys
    torch.cuda.synchronize()
    for a, b in zip(out[FEW], out[MANY]):
        assert torch.equal(bits(a), bits(b[:FEW]))
