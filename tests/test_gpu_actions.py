"""Action-level parity at the full expert shape: the pi0.5-shaped action expert (18 layers; q 2048x1024, k/v 256x1024,
o 1024x2048, gate/up 4096x1024, down 1024x4096) with an 800-row prefix KV cache per observation and 10 Euler steps per
chunk.

  test_actions_over_observations   parity.py:81-102 (stage_actions): final actions on 40 observations with one fixed noise,
                                   every runtime against the W2A8 reference runtime; the kernel runtimes must agree on every
                                   observation bit for bit, the float rows (FP16 table, W2 float path, dense W2) are
                                   reported for scale and bounded.
  test_full_chunk_through_the_oracle   one whole chunk with every quantized layer call (126 layers x 10 steps) computed by
                                   the oracle's reference_linear on the host, equal bit for bit to the fused runtime's.

Observations here are synthetic: per observation, per-layer prefix keys / values drawn from N(0, 1) (the backbone's prefill
output in the policy)."""
import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'
LAYERS, PREFIX, STEPS, OBS = 18, 800, 10, 40


@pytest.fixture(scope='module', autouse=True)
def _lib():
    from yanlongvla_amd import _lib
    _lib.lib()
    torch.cuda.init()


def observation(i):
    g = torch.Generator(device=DEV).manual_seed(1000 + i)
    ks = [torch.randn(PREFIX, 256, generator=g, device=DEV).bfloat16() for _ in range(LAYERS)]
    vs = [torch.randn(PREFIX, 256, generator=g, device=DEV).bfloat16() for _ in range(LAYERS)]
    return ks, vs


def noise():
    return torch.randn(50, 32, generator=torch.Generator(device=DEV).manual_seed(0), device=DEV)


def expert(**install):
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.ExpertPolicy, DEV, seed=21, layers=LAYERS)
    info = modules.install(model, layers=gemma.synthetic_layers(model, 22, DEV), **install) if install else None
    return model, info


ROWS = dict(w2a8_ref=dict(runtime='reference'), w2a8_resident=dict(runtime='resident'), w2a8_fly=dict(runtime='fly'),
            w2a8_hybrid=dict(runtime='hybrid'), w2a8_ref_fp16table=dict(runtime='reference', table='fp16'),
            w2_ref=dict(runtime='reference', a8=False), w2_fly=dict(runtime='fly', a8=False), w2_dense=dict(runtime='dense'))


@torch.no_grad()
def test_actions_over_observations():
    from yanlongvla_amd import harness, modules
    nz = noise()
    acts = {}
    for row, kw in ROWS.items():
        model, info = expert(**kw)
        assert info['layers'] == 7 * LAYERS
        a = []
        for i in range(OBS):
            model.set_prefix(*observation(i))
            modules.decode_chunk(model)
            a.append(model.sample_chunk(nz, steps=STEPS).float().cpu().numpy())
        acts[row] = np.stack(a)
        del model
        torch.cuda.empty_cache()
    table = harness.action_table(acts, 'w2a8_ref')
    for row, t in table.items():
        print(f"{row:20s} identical {t['identical_observations']:2d}/{OBS}  max|dA| {t['max_abs']:.3e}  "
              f"rel err max {t['rel_err_max']:.3e}  mean {t['rel_err_mean']:.3e}", flush=True)
    assert all(np.isfinite(a).all() for a in acts.values())
    for row in ('w2a8_resident', 'w2a8_fly', 'w2a8_hybrid'):
        assert table[row]['identical_observations'] == OBS, (row, table[row])
    # the distinct observations give distinct actions (the parity above is not over one repeated case)
    assert len({a.tobytes() for a in acts['w2a8_ref']}) == OBS
    # the W2 float path's kernels (BF16 rotated activations and products, modules.py:117-144) against the float
    # definition (FP32 activations, FP64 sums): per layer within 2e-3, here through 18 layers and 10 steps
    w2 = harness.action_table({r: acts[r] for r in ('w2_ref', 'w2_fly')}, 'w2_ref')['w2_fly']
    print(f"w2_fly vs w2_ref       rel err max {w2['rel_err_max']:.3e}  mean {w2['rel_err_mean']:.3e}", flush=True)
    assert w2['rel_err_max'] < 5e-3, w2                                  # measured 7.6e-4
    # the float rows stay near the W2A8 model: activation quantization is the only difference from the W2 model
    for row in ('w2a8_ref_fp16table', 'w2_ref', 'w2_dense'):
        assert table[row]['rel_err_max'] < 1e-2, (row, table[row])         # measured 8.3e-4 .. 8.7e-4


class OracleLinear(torch.nn.Module):
    """A quantized Linear computed on the host by the oracle (INT8 weights decoded once by the oracle)."""

    def __init__(self, layer):
        super().__init__()
        t = dict(bits=layer.bits.cpu().numpy(), tlut=layer.tlut.cpu().numpy(), row_scale=layer.row_scale.cpu().numpy(),
                 su=layer.su.cpu().numpy(), sv=layer.sv.cpu().numpy())
        self.ol = O.Layer(layer.name, t)
        self.w8 = self.ol.w8_reference()
        self.calls = 0

    def forward(self, x):
        self.calls += 1
        y = O.reference_linear(x.float().reshape(-1, self.ol.n).cpu().numpy(), self.ol, w8=self.w8)
        return torch.from_numpy(y.view(np.int16)).to(x.device).view(torch.bfloat16).reshape(*x.shape[:-1], self.ol.m)


@torch.no_grad()
def test_full_chunk_through_the_oracle():
    from yanlongvla_amd import gemma, modules
    nz = noise()
    ks, vs = observation(3)
    fly, info = expert(runtime='fly')
    assert info['fused_layers'] == LAYERS
    fly.set_prefix(ks, vs)
    want = fly.sample_chunk(nz, steps=STEPS)
    del fly
    torch.cuda.empty_cache()
    model, _ = expert()
    bridges = {}
    for name, layer in gemma.synthetic_layers(model, 22, DEV).items():
        bridges[name] = OracleLinear(layer)
        modules.set_submodule(model, name, bridges[name])
    model.set_prefix(ks, vs)
    got = model.sample_chunk(nz, steps=STEPS)
    assert len(bridges) == 7 * LAYERS and all(b.calls == STEPS for b in bridges.values())
    assert torch.equal(got, want)
