"""The op-level helpers with the reference's own signatures (deploy/tcq_kernels/kernels.py:602-696), called the way the
reference's Group calls them (deploy/tcq_kernels/modules.py:69-106): activations quantized into q4 (K/4, M) words,
the group's packed words as stored (bits of the members concatenated along the rows), their INT8 tables concatenated,
table bounds at the members' first tile rows, FP32 z (M, N) out, then post3 / postg on the concatenated row scales, signs
and biases. Every result goes through the C ABI and is compared with the oracle bit for bit."""
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


class RefShapedGroup:
    """What the reference's Group.__init__ keeps for an expert group (modules.py:30-46): concatenated rs / sv / bias, t8 and
    bits, and the tile-row bounds of the members."""

    def __init__(self, layers):
        from yanlongvla_amd import kernels as K
        self.layers = layers
        self.K = layers[0].n
        self.N = [L.m for L in layers]
        self.col0 = [sum(self.N[:i]) for i in range(len(layers))]
        self.Ntot = sum(self.N)
        self.rs_parts, t8s = [], []
        for L in layers:
            t8, rs, _ = K.snap(T(L.tlut.view(np.int16)), T(L.row_scale.view(np.int16)))
            t8s.append(t8)
            self.rs_parts.append(rs)
        self.rs = torch.cat(self.rs_parts).contiguous()
        self.sv = torch.cat([T(L.sv) for L in layers]).contiguous()
        self.bias = (torch.cat([T(L.bias) for L in layers]).contiguous() if layers[0].bias is not None else None)
        self.t8 = torch.cat([t.reshape(-1) for t in t8s]).contiguous()
        self.bits = torch.cat([T(L.bits) for L in layers]).contiguous()
        self.bounds = [c // 16 for c in self.col0[1:]] + [1 << 30] * (3 - len(layers))
        self.su = T(layers[0].su)
        W = torch.empty(self.Ntot, self.K, dtype=torch.int8, device=DEV)
        for L, c, t in zip(layers, self.col0, t8s):
            K.decode(T(L.bits), t, W[c:c + L.m])
        self.W = W


def _group(shapes, seed, bias):
    rng = np.random.default_rng(seed)
    su = np.where(rng.integers(0, 2, shapes[0][1]) > 0, 1, -1).astype(np.int8)
    layers = []
    for i, (m, n) in enumerate(shapes):
        L = O.random_layer(m, n, seed * 10 + i, bias=bias, per_layer_scale=False)
        L.su = su                                                      # group members share the input signs
        layers.append(L)
    return layers


@pytest.mark.parametrize('shapes,M,bias', [([(2048, 1024), (256, 1024), (256, 1024)], 10, False),
                                           ([(2048, 1024), (256, 1024), (256, 1024)], 50, True),
                                           ([(4096, 1024), (4096, 1024)], 10, False),
                                           ([(1024, 4096)], 33, True), ([(48, 80), (32, 80)], 1, False)])
def test_reference_shaped_products_and_epilogues(shapes, M, bias):
    from yanlongvla_amd import kernels as K
    layers = _group(shapes, 7 + M + len(shapes), bias)
    g = RefShapedGroup(layers)
    x = np.random.default_rng(M).standard_normal((M, g.K)).astype(np.float32)
    # Group.buffers / quantize of the expert (modules.py:69-79)
    b = dict(q4=torch.empty(g.K // 4, M, dtype=torch.int32, device=DEV), scale=torch.empty(M, dtype=torch.float32, device=DEV))
    K.pre(T(x).bfloat16(), g.su, **b)
    h = O.fwht(O.bf16_to_f32(O.bf16_bits(x)) * layers[0].su.astype(np.float32))
    q, s = O.quantize_tokens(h)
    assert np.array_equal(b['q4'].cpu().numpy(), O.q4_layout(q))
    # Group.product, expert: fly (gemm_tcq on the stored words) and resident (gemm_w8) (modules.py:87-93)
    z_fly = torch.full((M, g.Ntot), float('nan'), device=DEV)
    K.gemm_tcq(g.bits, g.t8, b['q4'], b['scale'], g.rs, z_fly, g.K, g.bounds)
    z_res = torch.full((M, g.Ntot), float('nan'), device=DEV)
    K.gemm_w8(g.W, b['q4'], b['scale'], g.rs, z_res)
    ref = np.concatenate([(O.int_matmul(q, L.w8_reference()).astype(np.float32) * s) * L.rs[None, :] for L in layers], 1)
    assert np.array_equal(z_fly.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(z_res.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    # Group.posts, expert (modules.py:95-106): FP32 z already scaled, so s and rs are None
    ys = [torch.empty(M, n, dtype=torch.bfloat16, device=DEV) for n in g.N]
    if len(ys) == 3:
        K.post3(z_fly, None, None, g.sv, g.bias, ys)
        ys2 = [torch.empty_like(y) for y in ys]
        K.postg(z_fly, None, None, g.sv, g.bias, ys2)
        assert all(torch.equal(a, c) for a, c in zip(ys, ys2))
    elif len(ys) == 2:
        K.postg(z_fly, None, None, g.sv, g.bias, ys)
    else:
        K.post(z_fly, None, None, g.sv, g.bias, ys[0], col0=0)
    for L, c, y in zip(layers, g.col0, ys):
        want = O.reference_linear(O.bf16_to_f32(O.bf16_bits(x)), L)
        assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), want)


def test_reference_shaped_gated_middle_split():
    """KGatedMLP's split middle for few tokens (modules.py:182-185): postg(acc, None, None, sv, None, [g, u], gelu0=True)
    then pre2 -> q4 / scale; equal to the fused mid2."""
    from yanlongvla_amd import kernels as K
    rng = np.random.default_rng(3)
    M, N = 10, 4096
    z = rng.standard_normal((M, 2 * N)).astype(np.float32)
    sv = np.where(rng.integers(0, 2, 2 * N) > 0, 1, -1).astype(np.int8)
    su = np.where(rng.integers(0, 2, N) > 0, 1, -1).astype(np.int8)
    g_ = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    u_ = torch.empty_like(g_)
    K.postg(T(z), None, None, T(sv), None, [g_, u_], gelu0=True)
    b2 = dict(q4=torch.empty(N // 4, M, dtype=torch.int32, device=DEV), scale=torch.empty(M, dtype=torch.float32, device=DEV))
    K.pre2(g_, u_, T(su), **b2)
    b3 = dict(q4=torch.empty(N // 4, M, dtype=torch.int32, device=DEV), scale=torch.empty(M, dtype=torch.float32, device=DEV))
    K.mid2(T(z), None, None, T(sv), T(su), **b3)
    assert torch.equal(b2['q4'], b3['q4']) and torch.equal(b2['scale'], b3['scale'])
    lut = K.gelu_table(DEV).view(torch.int16).cpu().numpy().view(np.uint16)
    qr, sr, gb, ub = O.mlp_middle(z[:, :N], z[:, N:], sv[:N], sv[N:], su, gelu=lambda v: lut[v])
    assert np.array_equal(g_.view(torch.int16).cpu().numpy().view(np.uint16), gb)
    assert np.array_equal(u_.view(torch.int16).cpu().numpy().view(np.uint16), ub)
    assert np.array_equal(b2['q4'].cpu().numpy(), O.q4_layout(qr)) and np.array_equal(b2['scale'].cpu().numpy(), sr[:, 0])


def test_reference_shaped_argument_errors():
    from yanlongvla_amd import kernels as K, _lib
    layers = _group([(64, 256)], 1, False)
    g = RefShapedGroup(layers)
    q4 = torch.zeros(64, 65, dtype=torch.int32, device=DEV)
    s = torch.ones(65, device=DEV)
    z = torch.empty(65, 64, device=DEV)
    with pytest.raises(_lib.TcqError):                          # 65 tokens: more than the small-M product takes
        K.gemm_w8(g.W, q4, s, g.rs, z)
    with pytest.raises(ValueError):                             # q4 of the wrong K
        K.gemm_w8(g.W, q4[:32], s, g.rs, z)
    with pytest.raises(ValueError):                             # bounds select a second table that is not there
        K.gemm_tcq(g.bits, g.t8, torch.zeros(64, 4, dtype=torch.int32, device=DEV), s, g.rs, z[:4], g.K, (2, 1 << 30))
