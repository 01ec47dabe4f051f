"""GPU tests of the multi-query attention kernel: against FP64 attention (the BF16 output rounding is the only sizeable
difference), causal visibility, the fused o-projection prologue against attention followed by the separate prologue, and
run-to-run determinism."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = 'cuda'


@pytest.fixture(scope='module', autouse=True)
def _lib():
    from yanlongvla_amd import _lib
    _lib.lib()
    torch.cuda.init()


def reference(q, kc, vc, kn, vn, H, causal):
    """FP64 softmax(q k^T / 16) v over cache + new rows; query t sees key j iff causal is None or j <= causal + t."""
    k = torch.cat([kc, kn]) if kc is not None else kn
    v = torch.cat([vc, vn]) if vc is not None else vn
    M, D = q.shape[0], k.shape[1]
    qh = q.double().cpu().reshape(M, H, D)
    s = torch.einsum('thd,jd->thj', qh, k.double().cpu()) / 16.0
    if causal is not None:
        j = torch.arange(k.shape[0])[None, None, :]
        t = torch.arange(M)[:, None, None]
        s = s.masked_fill(j > t + causal, float('-inf'))
    p = torch.softmax(s, -1)
    return torch.einsum('thj,jd->thd', p, v.double().cpu()).reshape(M, H * D)


def inputs(M, P, H, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device=DEV).bfloat16()
    return r(M, H * 256), (r(P, 256) if P else None), (r(P, 256) if P else None), r(M, 256), r(M, 256)


@pytest.mark.parametrize('M,P,H,causal', [(50, 800, 8, None), (1, 832, 8, None), (800, 0, 8, 0), (7, 0, 8, 0), (3, 63, 4, None),
                                          (1, 0, 1, None), (65, 10, 8, 10)])
def test_attend_matches_fp64(M, P, H, causal):
    from yanlongvla_amd import kernels as K
    q, kc, vc, kn, vn = inputs(M, P, H, M + P + H)
    o = torch.empty(M, H * 256, dtype=torch.bfloat16, device=DEV)
    K.attend(q, kc, vc, kn, vn, H, causal, o=o)
    ref = reference(q, kc, vc, kn, vn, H, causal)
    got = o.double().cpu()
    assert torch.isfinite(got).all()
    assert ((got - ref).norm() / ref.norm()).item() < 4e-3
    assert (got - ref).abs().max().item() < 2e-2 * ref.abs().max().item() + 1e-3


def test_causal_rows_ignore_later_keys():
    """Changing the keys / values a causal query may not see leaves its output unchanged."""
    from yanlongvla_amd import kernels as K
    q, _, _, kn, vn = inputs(200, 0, 8, 3)
    o1 = torch.empty(200, 2048, dtype=torch.bfloat16, device=DEV)
    K.attend(q, None, None, kn, vn, 8, 0, o=o1)
    kn2, vn2 = kn.clone(), vn.clone()
    kn2[100:] = torch.randn_like(kn2[100:].float()).bfloat16()
    vn2[100:] = torch.randn_like(vn2[100:].float()).bfloat16()
    o2 = torch.empty_like(o1)
    K.attend(q, None, None, kn2, vn2, 8, 0, o=o2)
    assert torch.equal(o1[:100], o2[:100]) and not torch.equal(o1[100:], o2[100:])


@pytest.mark.parametrize('H', [1, 2, 4, 8])
@pytest.mark.parametrize('M,P,causal', [(50, 800, None), (1, 800, None), (300, 0, 0), (7, 0, 0), (20, 40, 40)])
def test_fused_prologue_bitexact(M, P, causal, H):
    """The o-projection prologue fused into attention (rotate + quantize of the BF16 attention output, every engine width
    H * 256 = 256 .. 2048) equals attention followed by kernels.pre bit for bit: q8, the token-block q4 and the scales.
    Cases: a prefix without masking, a causal prefill with no prefix, and causal rows over a prefix (causal offset P)."""
    from yanlongvla_amd import kernels as K
    q, kc, vc, kn, vn = inputs(M, P, H, 7 + M + H)
    W = H * 256
    su = (torch.randint(0, 2, (W,), generator=torch.Generator(device=DEV).manual_seed(H), device=DEV) * 2 - 1).to(torch.int8)
    o = torch.empty(M, W, dtype=torch.bfloat16, device=DEV)
    K.attend(q, kc, vc, kn, vn, H, causal, o=o)
    q1, s1, tb1 = torch.empty(M, W, dtype=torch.int8, device=DEV), torch.empty(M, device=DEV), K.token_blocks(M, W, DEV)
    K.pre(o, su, q=q1, q4=tb1, scale=s1)
    q2, s2, tb2 = torch.empty_like(q1), torch.empty_like(s1), K.token_blocks(M, W, DEV)
    K.attend(q, kc, vc, kn, vn, H, causal, su=su, q8=q2, scale=s2, q4=tb2)
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    assert torch.equal(K.rows_of_token_blocks(tb1, M), K.rows_of_token_blocks(tb2, M))
    o2 = torch.empty_like(o)
    K.attend(q, kc, vc, kn, vn, H, causal, o=o2)
    assert torch.equal(o, o2)
