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
