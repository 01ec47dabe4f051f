"""Host-side logic that needs no GPU: layer naming and grouping rules, block widths, the packed file schema."""
import numpy as np
import pytest
import torch

from yanlongvla_amd import gemma, modules
from yanlongvla_amd import tcq_format as F


def quantizable(model):
    return [n for n, m in model.named_modules() if modules.is_quantizable(n, m)]


def test_expert_and_backbone_layer_sets():
    """The synthetic stacks carry the policy's quantizable layers: 126 expert layers holding 311,427,072 weights and 126
    language-model layers holding 1,981,808,640 (the pi0.5 counts)."""
    with torch.device('meta'):
        e, b = gemma.ExpertPolicy(), gemma.BackbonePolicy()
    for mdl, parts, count in ((e, {'expert'}, 311_427_072), (b, {'llm'}, 1_981_808_640)):
        names = quantizable(mdl)
        assert len(names) == 126
        assert {modules.part_of(n) for n in names} == parts
        assert sum(mdl.get_submodule(n).weight.numel() for n in names) == count
    assert not modules.is_quantizable('x.gemma_expert.model.layers.0.input_layernorm.dense', torch.nn.Linear(4, 4))
    assert not modules.is_quantizable('action_in_proj', e.action_in_proj)


def test_block_widths():
    assert F.block_widths(4304) == [4096, 128, 64, 16]
    assert F.block_widths(16384) == [16384]
    assert F.block_widths(1152) == [1024, 128]
    assert F.block_widths(0) == []


def test_packed_file_schema(tmp_path):
    rng = np.random.default_rng(0)
    t = dict(bits=torch.from_numpy(rng.integers(-32768, 32768, (4, 32)).astype(np.int16)),
             tlut=torch.randn(512, 2).half(), row_scale=torch.rand(32).half(),
             su=torch.ones(32, dtype=torch.int8), sv=-torch.ones(32, dtype=torch.int8))
    p = F.save({'a.b.q_proj': t, 'a.b.k_proj': t}, tmp_path / 'row' / 'packed.safetensors')
    assert F.packed_path(p) == p
    assert sorted(F.layer_names(p)) == ['a.b.k_proj', 'a.b.q_proj']
    from safetensors import safe_open
    with safe_open(str(p), framework='pt') as f:
        assert set(f.keys()) == {f'{n}::{k}' for n in ('a.b.q_proj', 'a.b.k_proj') for k in F.TENSORS}
        assert f.get_tensor('a.b.q_proj::bits').dtype == torch.int16
        assert torch.equal(f.get_tensor('a.b.q_proj::bits'), t['bits'])


def test_runtime_names_are_checked():
    with pytest.raises(ValueError):
        modules.install(torch.nn.Linear(2, 2), runtime='fast', layers={})


def test_from_qtip_matches_qtip_reconstruction(tmp_path):
    """The packed tensors converted from a QTIP-official record give, through the oracle's dense weight, QTIP's own inverse
    transform W = (hadU((hadU(Wscale Q) * SU)^T) * SV)^T with the normalised Sylvester Hadamard (quantize_qtip.py:72-74)."""
    from safetensors.torch import save_file
    from oracle import tcq_oracle as O
    rng = np.random.default_rng(9)
    m, n = 64, 128
    bits = rng.integers(-32768, 32768, ((m // 16) * (n // 16), 32)).astype(np.int16)
    tlut = rng.standard_normal((512, 2)).astype(np.float16)
    su = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    sv = np.where(rng.random(m) < 0.5, -1.0, 1.0).astype(np.float16)
    wscale = np.float32(0.0625)                                              # exact in FP16
    rec = dict(trellis_int16=torch.from_numpy(bits.reshape(-1)), tlut_fp16=torch.from_numpy(tlut),
               su_fp16=torch.from_numpy(su), sv_fp16=torch.from_numpy(sv), wscale_fp32=torch.tensor([wscale]))
    save_file(rec, str(tmp_path / 'q.safetensors'))
    p = F.convert_qtip({'l.q_proj': tmp_path / 'q.safetensors'}, tmp_path / 'packed.safetensors')
    from safetensors import safe_open
    with safe_open(str(p), framework='pt') as f:
        t = {k: f.get_tensor(f'l.q_proj::{k}').numpy() for k in F.TENSORS}
    L = O.Layer('l.q_proj', t)

    def H(k):
        h = np.ones((1, 1))
        while h.shape[0] < k:
            h = np.block([[h, h], [h, -h]])
        return h / np.sqrt(k)
    Q = O.lookup(L.states(), tlut.astype(np.float32)).astype(np.float64)
    hadU = lambda X: X @ H(X.shape[-1]).T
    W = (hadU((hadU(wscale * Q) * su.astype(np.float64)).T) * sv.astype(np.float64)).T
    assert np.allclose(L.dense('fp16'), W, atol=1e-5 * np.abs(W).max())
    with pytest.raises(ValueError):
        F.from_qtip(dict(rec, su_fp16=torch.ones(4480, dtype=torch.float16), trellis_int16=torch.zeros(4, 32, dtype=torch.int16)))


def test_decoder_layer_handoff_rules():
    """The chained prologue is taken only for the very tensor it was computed from (a view of it is fine), unmodified,
    and only once; for inference tensors (no version counter) only for the very object the previous layer returned."""
    import torch
    from yanlongvla_amd.modules import KDecoderLayer
    layer = KDecoderLayer.__new__(KDecoderLayer)
    torch.nn.Module.__init__(layer)
    b = dict(q=torch.zeros(4, 8, dtype=torch.int8), scale=torch.zeros(4))

    def hand(x4):
        out = x4.reshape(2, 2, 8)
        layer._handoff = (x4, None if x4.is_inference() else x4._version, out, b)
        return out

    def take(x):
        return layer._prologue(x, x.reshape(-1, 8).contiguous())

    x4 = torch.zeros(4, 8, dtype=torch.bfloat16)
    out = hand(x4)
    assert take(out) is b
    assert take(out) is None                                     # taken once
    out = hand(x4)
    assert take(x4) is b                                         # another view of the same storage, unmodified
    out = hand(x4)
    out.add_(1)
    assert take(out) is None                                     # modified in place since
    out = hand(x4)
    assert take(out.clone()) is None                             # another tensor with equal values
    out = hand(x4)
    assert layer._prologue(out, x4[:2]) is None                  # another shape
    with torch.inference_mode():
        y4 = torch.zeros(4, 8, dtype=torch.bfloat16)
        out = hand(y4)
        assert take(out) is b                                    # the returned object itself
        out = hand(y4)
        assert take(out + 0) is None                             # a new tensor
        out = hand(y4)
        assert take(y4.reshape(2, 2, 8)) is None                 # another object over the same storage


def test_groot_skeleton_matches_the_rule_accounting():
    """The GR00T skeleton's layers under GR00T's rule: 432 quantized Linear (216 backbone, 216 action head) holding
    2,340,421,632 weights, the reference's own accounting (groot_common.py:38-42); AdaLN linears, proj_out_*, lm_head and
    embeddings stay dense."""
    from yanlongvla_amd import groot, modules
    model = groot.skeleton()
    assert modules.rule_for(model) is modules.GROOT
    q = {n: m for n, m in model.named_modules() if modules.groot_is_quantizable(n, m)}
    assert len(q) == groot.QUANTIZED_LAYERS == 432
    assert sum(modules.groot_part_of(n) == 'backbone' for n in q) == 216
    assert sum(m.weight.numel() for m in q.values()) == groot.QUANTIZED_PARAMETERS == 2_340_421_632
    dense = [n for n, m in model.named_modules() if isinstance(m, torch.nn.Linear) and n not in q]
    assert sorted(dense) == sorted([f'action_head.model.transformer_blocks.{i}.norm1.linear' for i in range(32)] +
                                   ['action_head.model.proj_out_1', 'action_head.model.proj_out_2', 'backbone.model.lm_head'])
    assert not any(modules.is_quantizable(n, m) for n, m in q.items() if 'language_model' not in n)   # pi0.5's rule differs


def test_groot_group_plan():
    """Self-attention q/k/v (LLM, vl_self_attention, odd DiT blocks) and gate/up share a rotation; the cross-attention
    blocks' to_k / to_v read another width than to_q and stay single: 344 groups for 432 layers."""
    from types import SimpleNamespace
    from yanlongvla_amd import groot, modules
    model = groot.skeleton()
    signs = {}
    layers = {}
    for n, m in model.named_modules():
        if modules.groot_is_quantizable(n, m):
            w = m.in_features
            signs.setdefault(w, torch.ones(w, dtype=torch.int8))
            layers[n] = SimpleNamespace(n=w, su=signs[w], col_scale=None)
    plan = modules.plan_groups(list(layers), layers, modules.GROOT.families)
    assert len(plan) == 344 and sum(len(g) for g in plan) == 432
    assert ['backbone.model.model.language_model.layers.3.self_attn.q_proj', 'backbone.model.model.language_model.layers.3.self_attn.k_proj',
            'backbone.model.model.language_model.layers.3.self_attn.v_proj'] in plan
    cross = 'action_head.model.transformer_blocks.0.attn1.'
    assert [cross + 'to_k'] in plan and [cross + 'to_q'] in plan
    self_attn = 'action_head.model.transformer_blocks.1.attn1.'
    assert [self_attn + 'to_q', self_attn + 'to_k', self_attn + 'to_v'] in plan


def test_k_parts_rule():
    """K parts of a small-M product (Group.k_parts): doubled, up to 4, while the workgroups (one per tile row and part) stay
    below the 256 CUs and every part would keep at least 4 of the 256-column chunks; one part for many tokens or when off."""
    class G:
        pass

    def parts(n_out, k, m):
        g = G()
        g.Ntot, g.K = n_out, k
        return modules.Group.k_parts(g, m)
    assert parts(2048, 16384, 1) == 2           # backbone down: 128 tile rows x 2 parts = 256 workgroups
    assert parts(2048, 2048, 1) == 2            # backbone o
    assert parts(1024, 4096, 50) == 4           # expert down: 64 tile rows, 16 chunks
    assert parts(1024, 2048, 50) == 2           # expert o: 8 chunks allow one split
    assert parts(32768, 2048, 1) == 1           # gate/up: 2048 tile rows already fill the chip
    assert parts(256, 512, 3) == 1              # 2 chunks: no part would keep enough
    assert parts(2048, 16384, modules.SMALL_M + 1) == 1
    assert parts(1536, 6144, 1) == 1            # not a power of two: the epilogue takes no K parts at this width
    assert parts(512, 8192, 1) == 1             # below the epilogue's 1024-wide rows
    assert parts(1024, 8192, 1) == 4            # 64 tile rows, 32 chunks
    old = modules.FUSE['k_parts']
    modules.FUSE['k_parts'] = False
    try:
        assert parts(2048, 16384, 1) == 1
    finally:
        modules.FUSE['k_parts'] = old
