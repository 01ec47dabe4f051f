"""GR00T N1.7 drop-in on the GPU: install swaps the 432 quantized Linear layers of a GR00T-named model, and the GR00T record
forms -- one-sided layers (no output rotation) and column scales, with row-group tables -- are bit-exact against the
oracle through the fused runtime and through the layer-by-layer reference runtime."""
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


def oracle_layer(L):
    t = dict(bits=L.bits.cpu().numpy(), tlut=L.tlut.cpu().numpy(), row_scale=L.row_scale.cpu().numpy(), su=L.su.cpu().numpy())
    if L.sv is not None:
        t['sv'] = L.sv.cpu().numpy()
    if L.col_scale is not None:
        t['col_scale'] = L.col_scale.cpu().numpy()
    return O.Layer(L.name, t, bias=None if L.bias is None else L.bias.cpu().numpy())


def test_install_swaps_the_432_layers():
    from yanlongvla_amd import groot, modules
    model = groot.skeleton()
    layers = groot.synthetic_layers(model, 1, DEV)
    info = modules.install(model, runtime='fly', layers=layers)
    assert info['policy'] == 'gr00t' and info['layers'] == 432 and info['parts'] == {'backbone': 216, 'head': 216}
    assert info['groups'] == 344 and info['shared_rotations'] == 88
    swapped = [n for n, m in model.named_modules() if isinstance(m, modules.KLinear)]
    assert len(swapped) == 432
    assert all(L.sv is None and L.col_scale is not None for L in layers.values())
    del model, layers
    torch.cuda.empty_cache()


SAMPLE = ['backbone.model.model.visual.blocks.5.attn.qkv',                      # 3072 x 1024, 16 row-group tables
          'backbone.model.model.language_model.layers.2.self_attn.q_proj',      # q / k / v group, 2048 / 1024 / 1024 x 2048
          'backbone.model.model.language_model.layers.2.self_attn.k_proj',
          'backbone.model.model.language_model.layers.2.self_attn.v_proj',
          'backbone.model.model.language_model.layers.2.mlp.down_proj',         # 2048 x 6144 (4096 + 2048 block Walsh)
          'action_head.model.transformer_blocks.1.attn1.to_q',                  # self-attention group, 1536 x 1536
          'action_head.model.transformer_blocks.1.attn1.to_k',
          'action_head.model.transformer_blocks.1.attn1.to_v',
          'action_head.model.transformer_blocks.4.attn1.to_k',                  # cross-attention, 1536 x 2048
          'action_head.model.transformer_blocks.4.ff.net.0.proj',               # 6144 x 1536
          'action_head.model.transformer_blocks.4.ff.net.2']                    # 1536 x 6144


@pytest.mark.parametrize('one_sided', [True, False])
@pytest.mark.parametrize('runtime', ['fly', 'resident', 'reference'])
@pytest.mark.parametrize('M', [10, 100])
def test_groot_layers_bitexact(one_sided, runtime, M):
    """BF16 outputs of sampled GR00T layers, called as the model calls them (members of a group in turn on one input),
    equal the oracle's reference_linear bit for bit: few tokens on the fused small-M products, many on the INT8 GEMM."""
    from yanlongvla_amd import groot, modules
    model = groot.skeleton()
    layers = groot.synthetic_layers(model, 7 + M, DEV, one_sided=one_sided, names=SAMPLE)
    oracle = {n: oracle_layer(L) for n, L in layers.items()}
    modules.install(model, runtime=runtime, layers=layers)
    rng = np.random.default_rng(M)
    inputs = {}
    for name in SAMPLE:
        mod = model.get_submodule(name)
        n = mod.in_features
        parent = name.rpartition('.')[0]
        key = (parent, n)                                  # members of one group read one tensor
        if key not in inputs:
            inputs[key] = torch.from_numpy(rng.standard_normal((M, n)).astype(np.float32)).bfloat16().to(DEV)
        x = inputs[key]
        y = mod(x)
        want = O.reference_linear(x.float().cpu().numpy(), oracle[name])
        assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), want), name


@pytest.mark.parametrize('one_sided', [True, False])
def test_groot_fit_records_load_and_run(one_sided, tmp_path):
    """GR00T fit records as groot_tcq.py writes them (torch.save of {w_hat, tensors: trellis (uint16), tlut, row_scale,
    signs[, signs_out], col_scale, tcq}, 341-347 / 470-472), loaded by tcq_format.load_groot and installed: the layers'
    outputs at 10 tokens equal the oracle's reference_linear of the same records bit for bit (fly runtime)."""
    from yanlongvla_amd import groot, modules, tcq_format as F
    model = groot.skeleton()
    src = groot.synthetic_layers(model, 31, DEV, one_sided=one_sided, names=SAMPLE)
    files = {}
    for name, L in src.items():
        t = dict(trellis=L.bits.cpu().view(torch.uint16).reshape(-1), tlut=L.tlut.cpu(), row_scale=L.row_scale.cpu(),
                 signs=L.su.cpu(), col_scale=L.col_scale.cpu())
        if L.sv is not None:
            t['signs_out'] = L.sv.cpu()
        files[name] = tmp_path / f'{name}.pt'
        torch.save(dict(w_hat=torch.zeros(1), tensors=t, tcq=dict(L=16, K=2, V=2, td=16, rotation='one' if one_sided else 'two')),
                   files[name])
    oracle = {n: oracle_layer(L) for n, L in src.items()}
    biases = {n: L.bias for n, L in src.items() if L.bias is not None}      # the model's biases (records hold none)
    del src
    layers = F.load_groot(files, device=DEV, biases=biases)
    assert all((L.sv is None) == one_sided and L.col_scale is not None for L in layers.values())
    modules.install(model, runtime='fly', layers=layers)
    rng = np.random.default_rng(3)
    inputs = {}
    for name in SAMPLE:
        mod = model.get_submodule(name)
        key = (name.rpartition('.')[0], mod.in_features)
        if key not in inputs:
            inputs[key] = torch.from_numpy(rng.standard_normal((10, mod.in_features)).astype(np.float32)).bfloat16().to(DEV)
        y = mod(inputs[key])
        want = O.reference_linear(inputs[key].float().cpu().numpy(), oracle[name])
        assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), want), name
