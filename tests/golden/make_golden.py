"""Writes tests/golden/tcq_format_golden.npz: input/output vectors of the reference's own PyTorch arithmetic
(deploy/tcq_kernels/tcq_format.py), imported on the CPU from the reference checkout. Run once in a container that holds the
reference (the fixture file is committed; nothing under tests/ reads the reference at test time):

    python tests/golden/make_golden.py [/root/reference]

Cases are small and seeded. BF16 outputs are stored as int16 bit patterns, FP16 inputs as float16.
"""
import json
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path(sys.argv[1] if len(sys.argv) > 1 else '/root/reference') / 'deploy' / 'tcq_kernels'
sys.path.insert(0, str(REF))
import tcq_format as F  # noqa: E402  (the reference module, CPU only)

OUT = Path(__file__).with_name('tcq_format_golden.npz')


def layer_tensors(g, m, n, per_row_scale):
    bits = torch.randint(-32768, 32768, ((m // 16) * (n // 16), 32), generator=g, dtype=torch.int32).to(torch.int16)
    tlut = torch.randn(512, 2, generator=g).to(torch.float16)
    if per_row_scale:
        row_scale = (torch.rand(m, generator=g) + 0.5).to(torch.float16)
    else:
        row_scale = torch.full((m,), float(torch.rand(1, generator=g)) + 0.5).to(torch.float16)
    su = torch.where(torch.rand(n, generator=g) < 0.5, -1, 1).to(torch.int8)
    sv = torch.where(torch.rand(m, generator=g) < 0.5, -1, 1).to(torch.int8)
    return dict(bits=bits, tlut=tlut, row_scale=row_scale, su=su, sv=sv)


def main():
    g = torch.Generator().manual_seed(20261201)
    out = {}
    # block_widths
    widths = [1, 2, 3, 16, 48, 80, 1024, 1152, 1536, 4304, 6144]
    out['block_widths'] = np.array(json.dumps({str(w): F.block_widths(w) for w in widths}))
    # fwht, including non-power-of-two block decompositions
    for w in (1, 2, 16, 48, 80, 256, 1152, 4304):
        x = torch.randn(3, w, generator=g) * 2.0
        out[f'fwht_x_{w}'] = x.numpy()
        out[f'fwht_y_{w}'] = F.fwht(x).numpy()
    # exact-zero and repeated values (signed-zero behaviour of the butterflies)
    x = torch.zeros(2, 64)
    x[1, ::2] = 1.0
    x[1, 1::2] = 1.0
    out['fwht_x_ties'] = x.numpy()
    out['fwht_y_ties'] = F.fwht(x).numpy()
    # quantize_tokens: random rows, an all-zero row, a row of exact half-way quotients
    h = torch.randn(6, 64, generator=g) * 3
    h[2] = 0
    h[3] = torch.arange(64, dtype=torch.float32) - 31.5
    h[4, :] = torch.linspace(-1, 1, 64)
    q, s = F.quantize_tokens(h)
    out.update(qt_h=h.numpy(), qt_q=q.numpy(), qt_s=s.numpy())
    # int_matmul CPU branch
    a = torch.randint(-127, 128, (5, 64), generator=g, dtype=torch.int32).to(torch.int8)
    b = torch.randint(-127, 128, (24, 64), generator=g, dtype=torch.int32).to(torch.int8)
    out.update(im_a=a.numpy(), im_b=b.numpy(), im_acc=F.int_matmul(a, b).numpy())
    # layers: states, lookups, snap, w8, dense, reference_linear in every mode
    cases = [('l0', 32, 48, False, False), ('l1', 48, 80, True, True), ('l2', 64, 64, True, False), ('l3', 16, 256, False, True)]
    for tag, m, n, per_row, with_bias in cases:
        t = layer_tensors(g, m, n, per_row)
        bias = (torch.randn(m, generator=g) * 0.1) if with_bias else None
        L = F.Layer(tag, t, bias=bias, device='cpu')
        for k, v in t.items():
            out[f'{tag}_{k}'] = v.numpy()
        if bias is not None:
            out[f'{tag}_bias'] = bias.numpy()
        st = L.states()
        out[f'{tag}_states'] = st.to(torch.int32).numpy()
        out[f'{tag}_lookup_f32'] = F.lookup(st, L.tlut.float()).numpy()
        out[f'{tag}_t8'] = L.t8.numpy()
        out[f'{tag}_rs'] = L.rs.numpy()
        out[f'{tag}_gain'] = np.float32(L.gain)
        out[f'{tag}_w8'] = L.w8_reference().numpy()
        out[f'{tag}_dense_fp16'] = L.dense('fp16').numpy()
        out[f'{tag}_dense_int8'] = L.dense('int8').numpy()
        for dt in ('f32', 'bf16'):
            x = torch.randn(3, n, generator=g) * 2
            if dt == 'bf16':
                x = x.to(torch.bfloat16)
                out[f'{tag}_x_{dt}'] = x.view(torch.int16).numpy()
            else:
                out[f'{tag}_x_{dt}'] = x.numpy()
            for a8 in (True, False):
                for table in ('int8', 'fp16'):
                    y = F.reference_linear(x, L, a8=a8, table=table)
                    out[f'{tag}_y_{dt}_{"a8" if a8 else "a16"}_{table}'] = y.view(torch.int16).numpy()
                    yf = F.reference_linear(x, L, a8=a8, table=table, out_dtype=torch.float32)
                    out[f'{tag}_yf_{dt}_{"a8" if a8 else "a16"}_{table}'] = yf.numpy()
    # snap edge: a table whose amax entry is negative, and a tiny-magnitude table
    for tag, scale in (('snap_neg', -3.0), ('snap_tiny', 1e-3)):
        tl = torch.randn(512, 2, generator=g)
        tl[7, 1] = scale * 2.5
        tl = (tl * abs(scale)).to(torch.float16)
        rsc = (torch.rand(16, generator=g) + 0.5).to(torch.float16)
        t8, rs, gain = F.snap(tl, rsc)
        out.update({f'{tag}_tlut': tl.numpy(), f'{tag}_row_scale': rsc.numpy(), f'{tag}_t8': t8.numpy(), f'{tag}_rs': rs.numpy(),
                    f'{tag}_gain': np.float32(gain)})
    # GELU (tanh) of every BF16 bit pattern by PyTorch CPU (the routine the reference tabulates)
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    out['gelu_bf16_all'] = torch.nn.functional.gelu(allb, approximate='tanh').view(torch.int16).numpy()
    out['torch_version'] = np.array(torch.__version__)
    w2_integer_case(out)
    np.savez_compressed(OUT, **out)
    print(f'wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)')


def w2_integer_case(out):
    """reference_linear(a8=False, table='int8') on inputs whose rotated activations fwht(x * su) are exact integers (n = 256,
    where 1 / sqrt(256) is exact): x = su * fwht(v) for integer rows v with 64 <= |v| < 200. Also x_b, whose rotated
    activations are v + 1/32 (below half a BF16 ulp of v). Own generator, so the cases above keep their bytes."""
    g = torch.Generator().manual_seed(20261202)
    m, n = 64, 256
    t = layer_tensors(g, m, n, True)
    bias = torch.randn(m, generator=g) * 0.1
    L = F.Layer('w2i', t, bias=bias, device='cpu')
    mag = torch.randint(64, 200, (3, n), generator=g).float()
    v = torch.where(torch.rand(3, n, generator=g) < 0.5, -mag, mag)
    su = t['su'].float()
    x = F.fwht(v) * su
    xb = x.clone()
    xb[:, 0] += 0.5 * su[0]
    assert torch.equal(F.fwht(x * su), v), 'rotated activations are not the exact integers'
    assert torch.equal(F.fwht(xb * su), v + 1.0 / 32), 'offset rotated activations are not exact'
    for k, val in t.items():
        out[f'w2i_{k}'] = val.numpy()
    out.update(w2i_bias=bias.numpy(), w2i_v=v.numpy(), w2i_x=x.numpy(), w2i_xb=xb.numpy(), w2i_w8=L.w8_reference().numpy())
    out['w2i_y_bf16'] = F.reference_linear(x, L, a8=False, table='int8').view(torch.int16).numpy()
    out['w2i_y_f32'] = F.reference_linear(x, L, a8=False, table='int8', out_dtype=torch.float32).numpy()


if __name__ == '__main__':
    main()
