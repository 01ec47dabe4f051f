"""GPU parity of the RMSNorm kernel and its fusions (norm + rotate + quantize; epilogue + residual + norm + rotate +
quantize) against the oracle and against the unfused launches, and of the fused decoder layer against the module-by-module
forward."""
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


def bf16_dev(bits):
    return T(bits.view(np.int16)).view(torch.bfloat16)


def bits_of(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def signs(rng, n):
    return np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8)


@pytest.mark.parametrize('M,K', [(1, 1024), (50, 1024), (50, 2048), (800, 2048), (3, 16384), (5, 48)])
def test_rmsnorm_bitexact(M, K):
    from yanlongvla_amd import kernels as Kn
    rng = np.random.default_rng(M + K)
    x = O.bf16_bits(rng.standard_normal((M, K)).astype(np.float32) * 2)
    w = O.bf16_bits(rng.standard_normal(K).astype(np.float32) * 0.2)
    y = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    Kn.rmsnorm(bf16_dev(x), bf16_dev(w), 1e-6, y)
    assert np.array_equal(bits_of(y), O.rmsnorm_bf16(O.bf16_to_f32(x), w, 1e-6))


@pytest.mark.parametrize('M,K', [(1, 1024), (50, 1024), (800, 2048), (2, 16384)])
def test_norm_pre_bitexact(M, K):
    from yanlongvla_amd import kernels as Kn
    rng = np.random.default_rng(M * 3 + K)
    x = O.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = O.bf16_bits(rng.standard_normal(K).astype(np.float32) * 0.2)
    su = signs(rng, K)
    q = torch.empty(M, K, dtype=torch.int8, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    Kn.norm_pre(bf16_dev(x), bf16_dev(w), 1e-6, T(su), q=q, scale=s)
    qr, sr = O.quantize_tokens(O.fwht(O.bf16_to_f32(O.rmsnorm_bf16(O.bf16_to_f32(x), w, 1e-6)) * su.astype(np.float32)))
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr[:, 0])


@pytest.mark.parametrize('M,N,parts', [(1, 2048, 2), (50, 1024, 4), (3, 4096, 2), (2, 8192, 4), (1, 16384, 2)])
def test_post_add_norm_pre_k_parts(M, N, parts):
    """int32 K parts in: the same outputs as their int32 sum in one accumulator (register + transpose engine up to 4096,
    register engine beyond); a row the LDS path would take (N = 1152) is refused."""
    from yanlongvla_amd import kernels as Kn, _lib
    rng = np.random.default_rng(M + N + parts)
    lda = N + 64
    part = rng.integers(-2 ** 16, 2 ** 16, size=(parts, M, lda)).astype(np.int32)
    s = T((rng.random(M) * 1e-3 + 1e-4).astype(np.float32))
    rs = T((rng.random(N) * 1e-2).astype(np.float32))
    sv, su = T(signs(rng, N)), T(signs(rng, N))
    bias = T((rng.standard_normal(N) * 0.1).astype(np.float32))
    x = bf16_dev(O.bf16_bits(rng.standard_normal((M, N)).astype(np.float32)))
    w = bf16_dev(O.bf16_bits(rng.standard_normal(N).astype(np.float32) * 0.2))
    outs = []
    for acc in (T(part), T(part.sum(0, dtype=np.int32))):
        xo = torch.empty_like(x)
        q = torch.empty(M, N, dtype=torch.int8, device=DEV)
        sc = torch.empty(M, dtype=torch.float32, device=DEV)
        Kn.post_add_norm_pre(acc, s, rs, sv, bias, x, xo, w, 1e-6, su, q=q, scale=sc, col0=16)
        outs.append((xo, q, sc))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    with pytest.raises(_lib.TcqError):
        N2 = 1152
        acc = torch.zeros(parts, M, N2, dtype=torch.int32, device=DEV)
        xx = torch.zeros(M, N2, dtype=torch.bfloat16, device=DEV)
        Kn.post_add_norm_pre(acc, s, torch.ones(N2, device=DEV), T(signs(rng, N2)), None, xx, torch.empty_like(xx))


@pytest.mark.parametrize('kind', ['f32', 'i32'])
@pytest.mark.parametrize('M,N,col0', [(1, 1024, 16), (50, 1024, 16), (300, 2048, 16), (5, 4096, 16), (2, 16384, 16),
                                      (50, 1024, 2), (3, 4096, 2)])
@pytest.mark.parametrize('with_norm', [True, False])
def test_post_add_norm_pre_bitexact(kind, M, N, col0, with_norm):
    """== post (BF16) -> BF16 residual add -> rmsnorm -> pre, the unfused chain of launches. Aligned power-of-two rows
    run the register path (rows of 4096 and 16384 exchange between waves), col0 = 2 (rows not 16-byte aligned) the LDS
    path."""
    from yanlongvla_amd import kernels as Kn
    rng = np.random.default_rng(M * 5 + N)
    lda = N + 32
    if kind == 'i32':
        acc = T(rng.integers(-2 ** 18, 2 ** 18, size=(M, lda)).astype(np.int32))
        s = T((rng.random(M) * 1e-3 + 1e-4).astype(np.float32))
        rs = T((rng.random(N) * 1e-2).astype(np.float32))
    else:
        acc, s, rs = T(rng.standard_normal((M, lda)).astype(np.float32)), None, None
    sv, su = T(signs(rng, N)), T(signs(rng, N))
    bias = T((rng.standard_normal(N) * 0.1).astype(np.float32))
    x = bf16_dev(O.bf16_bits(rng.standard_normal((M, N)).astype(np.float32)))
    w = bf16_dev(O.bf16_bits(rng.standard_normal(N).astype(np.float32) * 0.2))
    xo = torch.empty_like(x)
    q = torch.empty(M, N, dtype=torch.int8, device=DEV)
    sc = torch.empty(M, dtype=torch.float32, device=DEV)
    if with_norm:
        Kn.post_add_norm_pre(acc, s, rs, sv, bias, x, xo, w, 1e-6, su, q=q, scale=sc, col0=col0)
    else:
        Kn.post_add_norm_pre(acc, s, rs, sv, bias, x, xo, col0=col0)
    a = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    Kn.post(acc, s, rs, sv, bias, a, col0=col0)
    x2 = x + a
    assert torch.equal(xo, x2)
    if with_norm:
        n = torch.empty_like(x2)
        Kn.rmsnorm(x2, w, 1e-6, n)
        q2 = torch.empty_like(q)
        s2 = torch.empty_like(sc)
        Kn.pre(n, su, q=q2, scale=s2)
        assert torch.equal(q, q2) and torch.equal(sc, s2)


def test_decoder_layer_fusion_is_bitexact():
    """KDecoderLayer (norms and residuals fused into the TCQ kernels) == the module-by-module forward (KLinear groups,
    KGatedMLP, device RMSNorm, PyTorch residual adds), at 50 tokens (small-M products) and 200 tokens (INT8 GEMM)."""
    from yanlongvla_amd import gemma, modules
    outs = {}
    for fuse in (False, True):
        old = modules.FUSE['layer']
        modules.FUSE['layer'] = fuse
        try:
            model = gemma.make_policy(gemma.ExpertPolicy, DEV, seed=1, layers=2)
            g = torch.Generator(device=DEV).manual_seed(2)
            model.set_prefix([torch.randn(64, 256, generator=g, device=DEV).bfloat16() for _ in range(2)],
                             [torch.randn(64, 256, generator=g, device=DEV).bfloat16() for _ in range(2)])
            with torch.no_grad():
                for n, p in model.named_parameters():
                    if n.endswith('layernorm.weight') or n.endswith('norm.weight'):
                        p.copy_((torch.randn(p.shape, generator=g, device=DEV) * 0.1).bfloat16())
            info = modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, 3, DEV))
            assert info['fused_layers'] == (2 if fuse else 0)
            if fuse:
                assert type(model.stack.layers[0]).__name__ == 'KDecoderLayer'
            x = torch.randn(50, 32, generator=torch.Generator(device=DEV).manual_seed(4), device=DEV)
            h = torch.randn(200, 1024, generator=torch.Generator(device=DEV).manual_seed(6), device=DEV).bfloat16()
            with torch.inference_mode():
                outs[fuse] = (model.velocity(x), model.stack.layers[1](h, model.prefix_k[1], model.prefix_v[1])[0])
        finally:
            modules.FUSE['layer'] = old
    assert torch.equal(outs[True][0], outs[False][0])
    assert torch.equal(outs[True][1], outs[False][1])
