"""Model-level parity of the Gemma-2B-shaped backbone at its full shape (18 layers; q / o 2048x2048, k / v 256x2048,
gate / up 16384x2048, down 2048x16384) against the oracle, as deploy/tcq_kernels/parity.py:22-73 checks every layer of a
policy forward on its in-model inputs: an 800-token causal prefill (256 image embeddings + 544 token embeddings), then
decode steps on the grown KV cache (decode_step_cached).

  test_backbone_through_the_oracle   the same model with every quantized Linear (126 layers) computed on the host by the
                                     oracle's reference_linear (tcq_format.py:125-148; INT8 weights decoded by the oracle)
                                     equals the fused fly and resident runtimes bit for bit: the prefill's last hidden
                                     state, every decode step's hidden state and every layer's KV cache rows.

The decoder layers' own operations (RMSNorm, attention, residual adds) run on the device kernels on both sides, as in
the expert's chunk test (test_gpu_actions.py)."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from oracle import tcq_oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'
LAYERS, IMAGE, TEXT, DECODE = 18, 256, 544, 2
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.fixture(scope='module', autouse=True)
def _lib():
    from yanlongvla_amd import _lib
    _lib.lib()
    torch.cuda.init()


def oracle_w8(ol, pool):
    """The oracle's INT8 weights of layer ol (Layer.w8_reference), decoded 64 tile rows at a time on a thread pool: tile
    rows are independent streams (states_from_bits reads tile row I from bits[I * n/16 : (I + 1) * n/16]), so the pieces
    are the whole decode."""
    n16, tr = ol.n // 16, ol.m // 16
    out = np.empty((ol.m, ol.n), np.int8)
    t16 = ol.t8.astype(np.int16)

    def rows(a):
        b = min(tr, a + 64)
        out[16 * a:16 * b] = O.lookup(O.states_from_bits(ol.bits[a * n16:b * n16], 16 * (b - a), ol.n), t16).astype(np.int8)
    list(pool.map(rows, range(0, tr, 64)))
    return out


class OracleLinear(torch.nn.Module):
    """A quantized Linear computed on the host by the oracle's reference_linear (W2A8, INT8 table, BF16 out)."""

    def __init__(self, layer, pool):
        super().__init__()
        t = dict(bits=layer.bits.cpu().numpy(), tlut=layer.tlut.cpu().numpy(), row_scale=layer.row_scale.cpu().numpy(),
                 su=layer.su.cpu().numpy(), sv=layer.sv.cpu().numpy())
        self.ol = O.Layer(layer.name, t)
        self.w8 = oracle_w8(self.ol, pool)
        self.calls = 0

    def forward(self, x):
        self.calls += 1
        y = O.reference_linear(x.float().reshape(-1, self.ol.n).cpu().numpy(), self.ol, w8=self.w8)
        return torch.from_numpy(y.view(np.int16)).to(x.device).view(torch.bfloat16).reshape(*x.shape[:-1], self.ol.m)


def inputs(model):
    g = torch.Generator(device=DEV).manual_seed(31)
    img = torch.randn(IMAGE, 2048, generator=g, device=DEV).bfloat16()
    ids = torch.randint(0, 1024, (TEXT,), generator=g, device=DEV)
    dec = torch.randint(0, 1024, (DECODE, 1), generator=g, device=DEV)
    return torch.cat([img, model.embed(ids)], 0), [model.embed(dec[t]) for t in range(DECODE)]


def run(model):
    """Prefill, then DECODE single-token steps on a KV cache: (prefill hidden state, decode hidden states, cache rows)."""
    from yanlongvla_amd import gemma
    x, dec = inputs(model)
    h, ks, vs = model.prefill(x)
    cache = gemma.KVCache(ks, vs, DECODE)
    hs = torch.cat([model.decode_step_cached(d, cache) for d in dec], 0)
    P = cache.length
    return h, hs, [k[:P] for k in cache.k], [v[:P] for v in cache.v]


def policy():
    from yanlongvla_amd import gemma
    return gemma.make_policy(gemma.BackbonePolicy, DEV, seed=32, layers=LAYERS, vocab=1024)


@torch.no_grad()
def test_backbone_through_the_oracle():
    from yanlongvla_amd import gemma, modules
    got = {}
    for runtime in ('fly', 'resident'):
        model = policy()
        info = modules.install(model, runtime=runtime, layers=gemma.synthetic_layers(model, 33, DEV))
        assert info['layers'] == 7 * LAYERS and info['fused_layers'] == LAYERS
        got[runtime] = [t.clone() if torch.is_tensor(t) else [u.clone() for u in t] for t in run(model)]
        del model
        torch.cuda.empty_cache()
    model = policy()
    bridges = {}
    with ThreadPoolExecutor(THREADS) as pool:
        for name, layer in gemma.synthetic_layers(model, 33, DEV).items():
            bridges[name] = OracleLinear(layer, pool)
            modules.set_submodule(model, name, bridges[name])
    want = run(model)
    assert len(bridges) == 7 * LAYERS and all(b.calls == 1 + DECODE for b in bridges.values())
    assert len({want[1][t].view(torch.int16).cpu().numpy().tobytes() for t in range(DECODE)}) == DECODE   # distinct steps
    for runtime, (h, hs, ks, vs) in got.items():
        assert torch.equal(h, want[0]), (runtime, 'prefill hidden state')
        assert torch.equal(hs, want[1]), (runtime, 'decode hidden states')
        bad = [i for i in range(LAYERS) if not (torch.equal(ks[i], want[2][i]) and torch.equal(vs[i], want[3][i]))]
        assert not bad, (runtime, 'KV cache rows of layers', bad)
