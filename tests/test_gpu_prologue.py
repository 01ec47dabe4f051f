"""GPU tests of the one-token products that run their activations' prologue in their own launch (tcq_gemm_tcq_pro /
tcq_gemm_w8_pro): every output equals, bit for bit, the standalone prologue kernel followed by the plain product on its
INT8 row. The decoder-layer prologue (tcq_post_add_norm_pre, 2048 wide): the residual output, the INT8 row and scale
copies, the FP32 z or the stage-split zt; the workgroup plan with one and two tile rows per workgroup, the streaming plan at
8 / 4 / 2 / 1 waves per tile row, the stage-split gate | up output; accumulators in one, two and four K parts. The rotate +
quantize prologue (tcq_pre, 16384 wide): int32 sums in one and two K parts on the streaming plan (fused decode) and the
workgroup plan (INT8-resident weights). The standalone kernels are pinned against the oracle in test_gpu_norms.py,
test_gpu_kernels.py and test_gpu_backbone_oracle.py."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = 'cuda'
K = 2048


@pytest.fixture(scope='module', autouse=True)
def _lib():
    from yanlongvla_amd import _lib
    _lib.lib()
    torch.cuda.init()


def signs(g, n):
    return (torch.randint(0, 2, (n,), generator=g, device=DEV) * 2 - 1).to(torch.int8)


def prologue_inputs(parts, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    shape = (parts, 1, K) if parts > 1 else (1, K)
    acc = torch.randint(-(1 << 20), 1 << 20, shape, generator=g, device=DEV, dtype=torch.int32)
    return dict(acc=acc, s=torch.rand(1, generator=g, device=DEV) * 1e-3 + 1e-4, rs=torch.rand(K, generator=g, device=DEV) * 1e-3,
                sv=signs(g, K), x=torch.randn(1, K, generator=g, device=DEV).bfloat16(),
                w=(torch.randn(K, generator=g, device=DEV) * 0.1).bfloat16(), eps=1e-6, su=signs(g, K))


def segments(widths, resident, seed, outs):
    from yanlongvla_amd import kernels as Kn
    g = torch.Generator(device=DEV).manual_seed(seed)
    segs = []
    for m, o in zip(widths, outs):
        rs = torch.rand(m, generator=g, device=DEV) * 1e-3
        if resident:
            w, t8 = torch.randint(-127, 128, (m, K), generator=g, device=DEV, dtype=torch.int8), None
        else:
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (Kn.repack_words(m, K),), generator=g, device=DEV, dtype=torch.int32)
            t8 = torch.randint(-127, 128, (512, 2), generator=g, device=DEV, dtype=torch.int8)
        segs.append((w, t8, rs, o))
    return segs


def reference_row(a):
    """tcq_post_add_norm_pre of the inputs: xout, the INT8 row and its scale."""
    from yanlongvla_amd import kernels as Kn
    xout = torch.empty_like(a['x'])
    q = torch.empty(1, K, dtype=torch.int8, device=DEV)
    sc = torch.empty(1, device=DEV)
    Kn.post_add_norm_pre(a['acc'], a['s'], a['rs'], a['sv'], None, a['x'], xout, a['w'], a['eps'], a['su'], q=q, scale=sc)
    return xout, q, sc


def pro_of(a):
    from yanlongvla_amd import kernels as Kn
    xout = torch.full_like(a['x'], float('nan'))
    q = torch.zeros(1, K, dtype=torch.int8, device=DEV)
    sc = torch.zeros(1, device=DEV)
    pro = Kn.prologue(a['acc'], a['s'], a['rs'], a['sv'], a['x'], xout, a['w'], a['eps'], a['su'], q=q, scale=sc)
    return pro, xout, q, sc


def bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32 if t.element_size() == 4 else torch.int8).cpu()


@pytest.mark.parametrize('widths,resident,parts', [
    ([2048, 256, 256], False, 2),          # workgroup plan, one tile row per workgroup (the backbone's q / k / v)
    ([2048, 256, 256], True, 1),
    ([16384, 16384], True, 2),             # workgroup plan, two tile rows (resident gate | up)
    ([16384, 16384], False, 4),            # streaming plan, 2 waves per tile row (fly gate | up)
    ([8192], False, 2),                    # 8 waves per tile row
    ([16384], False, 1),                   # 4
    ([65536], False, 2),                   # 1
])
def test_product_with_prologue_equals_the_two_launches(widths, resident, parts):
    from yanlongvla_amd import kernels as Kn
    a = prologue_inputs(parts, sum(widths) + parts)
    Ntot = sum(widths)
    cols = np.cumsum([0] + widths)[:-1]
    z_ref = torch.full((1, Ntot), float('nan'), device=DEV)
    z_pro = torch.full((1, Ntot), float('nan'), device=DEV)
    segs = segments(widths, resident, 7 + parts, [z_ref[:, c:] for c in cols])
    xout, q, sc = reference_row(a)
    Kn.SmallProduct(segs, Ntot, resident=resident)(q, sc)
    pro, xo2, q2, sc2 = pro_of(a)
    Kn.SmallProduct([(w, t8, rs, z_pro[:, c:]) for (w, t8, rs, _), c in zip(segs, cols)], Ntot, resident=resident).run_pro(pro)
    torch.cuda.synchronize()
    assert torch.equal(bits(xo2), bits(xout))
    assert torch.equal(q2.cpu(), q.cpu()) and torch.equal(bits(sc2), bits(sc))
    assert torch.equal(bits(z_pro), bits(z_ref))
    assert not torch.isnan(z_pro).any()


@pytest.mark.parametrize('parts', [1, 2])
def test_stage_split_middle_with_prologue(parts):
    """The gate | up product with the stage-split output (TCQ_Z_W128T) and the prologue: zt equals the two-launch form."""
    from yanlongvla_amd import kernels as Kn
    a = prologue_inputs(parts, 90 + parts)
    zt = [torch.full((2, 1, 128, 128), float('nan'), device=DEV) for _ in range(2)]
    segs = segments([16384, 16384], False, 11, [None, None])
    xout, q, sc = reference_row(a)
    Kn.gemm_tcq_w128t([(w, t8, rs, zt[0][i]) for i, (w, t8, rs, _) in enumerate(segs)], q, sc)
    pro, xo2, q2, sc2 = pro_of(a)
    Kn.gemm_tcq_w128t([(w, t8, rs, zt[1][i]) for i, (w, t8, rs, _) in enumerate(segs)], None, None, pro=pro)
    torch.cuda.synchronize()
    assert torch.equal(bits(xo2), bits(xout)) and torch.equal(q2.cpu(), q.cpu())
    assert torch.equal(bits(zt[1]), bits(zt[0]))
    assert not torch.isnan(zt[1]).any()


def test_prologue_refusals():
    """Layer prologues of rows other than 2048 wide or with int32 outputs, and rotate + quantize prologues of rows other
    than 16384 wide, are refused before any launch."""
    from yanlongvla_amd import kernels as Kn, _lib
    a = prologue_inputs(2, 5)
    z = torch.empty(1, 256, dtype=torch.int32, device=DEV)
    segs = segments([256], False, 3, [z])
    pro, _, _, _ = pro_of(a)
    with pytest.raises(_lib.TcqError):                                # int32 outputs after the layer prologue
        Kn.SmallProduct(segs, 256).run_pro(pro)
    with pytest.raises(_lib.TcqError):                                # a 2048-wide rotate + quantize prologue
        Kn.SmallProduct(segs, 256).run_pro(Kn.prologue_pre(a['x'], a['su']))
    z = torch.empty(1, 256, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(1, 1024, generator=g, device=DEV).bfloat16()
    pro1024 = Kn.prologue(a['acc'][:, :, :1024].contiguous(), a['s'], a['rs'][:1024].contiguous(), a['sv'][:1024].contiguous(), x,
                          torch.empty_like(x), a['w'][:1024].contiguous(), 1e-6, a['su'][:1024].contiguous())
    w = torch.randint(-127, 128, (256, 1024), generator=g, device=DEV, dtype=torch.int8)
    with pytest.raises(_lib.TcqError):                                # K = 1024: no variant
        Kn.SmallProduct([(w, None, segs[0][2], z)], 256, resident=True).run_pro(pro1024)


@pytest.mark.parametrize('resident,parts', [(False, 2), (False, 1), (True, 2), (True, 1)])
def test_product_with_rotate_quantize_prologue(resident, parts):
    """tcq_pre of a 16384-wide BF16 row inside the down projection's one-token product (2048 x 16384): the int32 sums, the
    INT8 row and the scale equal tcq_pre followed by the product."""
    from yanlongvla_amd import kernels as Kn
    Kd, m = 16384, 2048
    g = torch.Generator(device=DEV).manual_seed(40 + parts + 2 * resident)
    x = torch.randn(1, Kd, generator=g, device=DEV).bfloat16()
    su = signs(g, Kd)
    rs = torch.rand(m, generator=g, device=DEV) * 1e-3
    if resident:
        w, t8 = torch.randint(-127, 128, (m, Kd), generator=g, device=DEV, dtype=torch.int8), None
    else:
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (Kn.repack_words(m, Kd),), generator=g, device=DEV, dtype=torch.int32)
        t8 = torch.randint(-127, 128, (512, 2), generator=g, device=DEV, dtype=torch.int8)
    q = torch.empty(1, Kd, dtype=torch.int8, device=DEV)
    sc = torch.empty(1, device=DEV)
    Kn.pre(x, su, q=q, scale=sc)
    a_ref = torch.full((parts, 1, m), -5, dtype=torch.int32, device=DEV)
    Kn.SmallProduct([(w, t8, rs, a_ref[0])], m, resident=resident)(q, sc, parts)
    q2 = torch.zeros_like(q)
    sc2 = torch.zeros_like(sc)
    a_pro = torch.full((parts, 1, m), -7, dtype=torch.int32, device=DEV)
    Kn.SmallProduct([(w, t8, rs, a_pro[0])], m, resident=resident).run_pro(Kn.prologue_pre(x, su, q=q2, scale=sc2), parts)
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu(), q.cpu()) and torch.equal(bits(sc2), bits(sc))
    assert torch.equal(a_pro.cpu(), a_ref.cpu())


@pytest.mark.parametrize('resident,parts,P,causal', [(False, 2, 831, None), (True, 2, 831, None), (False, 1, 100, 100),
                                                     (True, 1, 64, 64), (False, 2, 2000, 1500)])
def test_product_with_attention_prologue(resident, parts, P, causal):
    """The attention's chunk merge + rotate + quantize (8 heads, one token against P cached keys) inside the o projection's
    product (2048 x 2048): the int32 sums, the INT8 row and the scale equal tcq_attend_q4's merge followed by the product;
    causal offsets that hide the last chunks (1500 of 2001 keys) included."""
    from yanlongvla_amd import kernels as Kn
    H, D, m = 8, 256, 2048
    g = torch.Generator(device=DEV).manual_seed(P + parts)
    q = torch.randn(1, H * D, generator=g, device=DEV).bfloat16()
    kc = torch.randn(P, D, generator=g, device=DEV).bfloat16()
    vc = torch.randn(P, D, generator=g, device=DEV).bfloat16()
    kn = torch.randn(1, D, generator=g, device=DEV).bfloat16()
    vn = torch.randn(1, D, generator=g, device=DEV).bfloat16()
    su = signs(g, H * D)
    (w, t8, rs, _), = segments([m], resident, 21 + P, [None])
    q8 = torch.empty(1, H * D, dtype=torch.int8, device=DEV)
    sc = torch.empty(1, device=DEV)
    Kn.attend(q, kc, vc, kn, vn, H, causal, su=su, q8=q8, scale=sc)
    a_ref = torch.full((parts, 1, m), -5, dtype=torch.int32, device=DEV)
    Kn.SmallProduct([(w, t8, rs, a_ref[0])], m, resident=resident)(q8, sc, parts)
    q2 = torch.zeros_like(q8)
    sc2 = torch.zeros_like(sc)
    a_pro = torch.full((parts, 1, m), -7, dtype=torch.int32, device=DEV)
    pro = Kn.prologue_attn(Kn.attend_parts(q, kc, vc, kn, vn, H, causal), H, su, q=q2, scale=sc2)
    Kn.SmallProduct([(w, t8, rs, a_pro[0])], m, resident=resident).run_pro(pro, parts)
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu(), q8.cpu()) and torch.equal(bits(sc2), bits(sc))
    assert torch.equal(a_pro.cpu(), a_ref.cpu())


@pytest.mark.parametrize('P,causal', [(831, None), (831, 831), (64, 64), (127, 127), (0, None), (2000, 1500)])
def test_attention_with_qkv_epilogue(P, causal):
    """tcq_attend_post_parts: the q / k / v epilogue of one FP32 product row (output rotations 2048 / 256 / 256 wide, signs,
    BF16) inside the attention's launch. The new key / value rows equal tcq_post_group's, and the chunk partials the merge
    reads (o, m, l of every visible chunk and head) equal tcq_attend_parts' on tcq_post_group's q / k / v, bit for bit: the
    new row first, last and inside its chunk, no cached rows, and a causal offset that hides the new row's chunk (its
    workgroup still writes the rows)."""
    from yanlongvla_amd import kernels as Kn
    H, D = 8, 256
    g = torch.Generator(device=DEV).manual_seed(P + 3)
    z = torch.randn(1, H * D + 2 * D, generator=g, device=DEV) * 3
    sv = signs(g, H * D + 2 * D)
    kc = torch.randn(P, D, generator=g, device=DEV).bfloat16() if P else None
    vc = torch.randn(P, D, generator=g, device=DEV).bfloat16() if P else None
    cols = [(0, H * D), (H * D, D), (H * D + D, D)]
    ys = [torch.empty(1, n, dtype=torch.bfloat16, device=DEV) for _, n in cols]
    Kn.post_group([(z, c0, None, sv[c0:c0 + n], None, y, False) for (c0, n), y in zip(cols, ys)], torch.float32, torch.bfloat16,
                  None, 1)
    part, nc, keys, cz = Kn.attend_parts(ys[0], kc, vc, ys[1], ys[2], H, causal)
    kn = torch.full((1, D), float('nan'), device=DEV).bfloat16()
    vn = torch.full((1, D), float('nan'), device=DEV).bfloat16()
    part2, nc2, keys2, cz2 = Kn.attend_post_parts(z, [(c0, sv[c0:c0 + n]) for c0, n in cols], kc, vc, kn, vn, H, causal)
    torch.cuda.synchronize()
    assert (nc2, keys2, cz2) == (nc, keys, cz)
    assert torch.equal(bits(kn), bits(ys[1])) and torch.equal(bits(vn), bits(ys[2]))
    T = P + 1
    nv = nc if causal is None else min(nc, (min(T, causal + 1) + 63) // 64)
    a = part.view(nc, H, D + 4)[:nv, :, :D + 2]
    b = part2.view(nc, H, D + 4)[:nv, :, :D + 2]
    assert torch.equal(bits(b), bits(a))
