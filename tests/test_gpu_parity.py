"""Stage-by-stage parity of every quantized layer on the inputs it receives inside a model, as deploy/tcq_kernels/parity.py
stage_layers does (parity.py:22-78): a Gemma-shaped stack installed with the reference runtime runs one forward with a hook on
every RefLinear; each layer's first input is then pushed through the device stages and compared bit for bit with the
oracle: decoded INT8 weights, INT8 activations, token scales, accumulators (exact int32 for the prefill product, FP32
z = (acc * s) * rs for the small-M fused and INT8-resident products) and BF16 outputs."""
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


def oracle_of(L):
    t = dict(bits=L.bits.cpu().numpy(), tlut=L.tlut.cpu().numpy(), row_scale=L.row_scale.cpu().numpy(),
             su=L.su.cpu().numpy(), sv=L.sv.cpu().numpy())
    return O.Layer(L.name, t, bias=None if L.bias is None else L.bias.cpu().numpy())


def stage_layers(model, run):
    from yanlongvla_amd import kernels as K
    from yanlongvla_amd.modules import RefLinear, SMALL_M
    seen = {}

    def hook(mod, inp, out):
        L = mod.layer[0]
        if L.name not in seen:
            seen[L.name] = (mod, inp[0].detach().clone(), out.detach().clone())

    handles = [m.register_forward_hook(hook) for m in model.modules() if isinstance(m, RefLinear)]
    with torch.inference_mode():
        run()
    for h in handles:
        h.remove()
    report = []
    for name, (mod, x, y_model) in seen.items():
        L = mod.layer[0]
        ol = oracle_of(L)
        x2 = x.reshape(-1, L.n).contiguous()
        M = x2.shape[0]
        h = O.fwht(x2.float().cpu().numpy() * ol.su.astype(np.float32))
        q_ref, s_ref = O.quantize_tokens(h)
        w8_ref = ol.w8_reference()
        acc_ref = O.int_matmul(q_ref, w8_ref)
        z_ref = (acc_ref.astype(np.float32) * s_ref) * ol.rs[None, :]
        y_ref = O.post_bf16(z_ref, ol.sv, ol.bias)
        rec = dict(name=name, tokens=M)
        rec['decode'] = np.array_equal(L.w8_reference().cpu().numpy(), w8_ref)
        q = torch.empty(M, L.n, dtype=torch.int8, device=DEV)
        s = torch.empty(M, device=DEV)
        K.pre(x2, L.su, q=q, scale=s)
        rec['activations'] = np.array_equal(q.cpu().numpy(), q_ref)
        rec['scales'] = np.array_equal(s.cpu().numpy(), s_ref[:, 0])
        if M <= SMALL_M:
            z1 = torch.empty(M, L.m, device=DEV)
            K.gemm_tcq_segments([(L.words(), L.t8, L.rs, z1)], q, s, L.m)
            z2 = torch.empty(M, L.m, device=DEV)
            K.gemm_w8_segments([(L.w8_reference(), None, L.rs, z2)], q, s, L.m)
            rec['accumulator'] = np.array_equal(z1.cpu().numpy().view(np.uint32), z_ref.view(np.uint32))
            rec['accumulator_resident'] = np.array_equal(z2.cpu().numpy().view(np.uint32), z_ref.view(np.uint32))
            acc, sa, rs = z1, None, None
        else:
            acc = K.gemm_i8(q, L.w8_reference(), torch.empty(M, L.m, dtype=torch.int32, device=DEV))
            rec['accumulator'] = np.array_equal(acc.cpu().numpy(), acc_ref)
            sa, rs = s, L.rs
        y = torch.empty(M, L.m, dtype=torch.bfloat16, device=DEV)
        K.post(acc, sa, rs, L.sv, L.bias, y)
        rec['output'] = np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), y_ref)
        rec['model_output'] = np.array_equal(y_model.reshape(M, L.m).contiguous().view(torch.int16).cpu().numpy().view(np.uint16),
                                             y_ref)
        report.append(rec)
    return report


def check(report, n_layers):
    keys = ('decode', 'activations', 'scales', 'accumulator', 'accumulator_resident', 'output', 'model_output')
    bad = [(r['name'], [k for k in keys if not r.get(k, True)]) for r in report]
    bad = [b for b in bad if b[1]]
    assert len(report) == n_layers and not bad, bad


def test_stage_layers_expert():
    """Every layer of a 2-layer expert at 50 action tokens (first flow step of a chunk)."""
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.ExpertPolicy, DEV, seed=3, layers=2)
    g = torch.Generator(device=DEV).manual_seed(4)
    model.set_prefix([torch.randn(128, 256, generator=g, device=DEV).bfloat16() for _ in range(2)],
                     [torch.randn(128, 256, generator=g, device=DEV).bfloat16() for _ in range(2)])
    modules.install(model, runtime='reference', layers=gemma.synthetic_layers(model, 5, DEV))
    noise = torch.randn(50, 32, generator=g, device=DEV)
    check(stage_layers(model, lambda: model.sample_chunk(noise, steps=1)), 14)


def test_stage_layers_backbone_prefill():
    """Every layer of a 2-layer backbone on a 200-token causal prefill (the INT8 MFMA GEMM path)."""
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.BackbonePolicy, DEV, seed=6, layers=2, vocab=1024)
    modules.install(model, runtime='reference', layers=gemma.synthetic_layers(model, 7, DEV))
    x = torch.randn(200, 2048, generator=torch.Generator(device=DEV).manual_seed(8), device=DEV).bfloat16()
    check(stage_layers(model, lambda: model.prefill(x)), 14)
