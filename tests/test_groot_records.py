"""GR00T TCQ fit records -> the deploy format (tcq_format.from_groot / convert_groot), on the CPU.

A record as baselines/groot/simpler/main_row/scripts/groot_tcq.py writes it (341-347 one- / two-sided bases, 470-472
row-group variants: `tensors` = trellis (uint16 words), tlut (512, 2) or (G, 512, 2), row_scale, signs[, signs_out]
[, col_scale]; `tcq` = the trellis settings) is built from random words and saved with torch.save. The converted layer's
dense weight (the oracle's Layer.dense, tcq_format.py:100-107) must equal GR00T's own decode of the record, restated here in
FP64 from groot_tcq.py: unpack's tile order (225-228), state_index / decode_normalized (143-175), the row and column
scales and inverse_rotation (178-191; inverse_rht = block Walsh then signs, groot_ptq.py:155-159). The record's states are
read from the words bit by bit (each 16 x 16 tile a 512-bit stream, most significant bit first; state t = bits
[4 t, 4 t + 16), tail-biting), the trellis QTIP's bitshift codebook packs (L = 16, K = 2, V = 2). Planted mistakes (swapped
sign vectors, the tile order without unpack's transpose, the column scale dropped) must fail.

Parity unpinned: that QTIP's pack_trellis lays its bits out as that stream (QTIP @ e90c6688 is not vendored); the
reference's own packer relies on the same identity for its pi0.5 records (deploy/tcq_kernels/tcq_format.py:204-207)."""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import tcq_oracle as O
from yanlongvla_amd import tcq_format as F


def record(m, n, seed, two_sided, col_scale, groups):
    g = torch.Generator().manual_seed(seed)
    words = torch.randint(0, 1 << 16, ((m // 16) * (n // 16), 32), generator=g, dtype=torch.int32).to(torch.uint16)
    tlut = torch.randn(*((groups,) if groups > 1 else ()), 512, 2, generator=g).half()
    t = dict(trellis=words.reshape(-1), tlut=tlut, row_scale=(torch.rand(m, generator=g) * 0.02 + 0.01).half(),
             signs=(torch.randint(0, 2, (n,), generator=g) * 2 - 1).to(torch.int8))
    if two_sided:
        t['signs_out'] = (torch.randint(0, 2, (m,), generator=g) * 2 - 1).to(torch.int8)
    if col_scale:
        t['col_scale'] = (torch.rand(n, generator=g) + 0.5).half()
    tcq = dict(L=16, K=2, V=2, tlut_bits=9, td=16, decode_mode='quantlut_sym', rotation='two' if two_sided else 'one')
    if groups > 1:
        tcq['groups'] = groups
    return dict(w_hat=torch.zeros(1), tensors=t, tcq=tcq)


def states_bit_by_bit(words):
    """(tiles, 32) uint16 -> (tiles, 128) states: state t = bits [4 t, 4 t + 16) of the tile's 512-bit stream (MSB first,
    tail-biting)."""
    w = words.astype(np.int64)
    stream = ((w[:, :, None] >> np.arange(15, -1, -1)) & 1).reshape(w.shape[0], 512)
    pos = (4 * np.arange(128)[:, None] + np.arange(16)[None, :]) % 512
    return (stream[:, pos] << (15 - np.arange(16))).sum(-1)


def block_hadamard(x):
    """Normalised block Walsh on the last axis in FP64: descending power-of-two blocks, Sylvester matrices / sqrt(w)."""
    out, off = [], 0
    for w in F.block_widths(x.shape[-1]):
        out.append(x[..., off:off + w] @ (scipy.linalg.hadamard(w).astype(np.float64) / math.sqrt(w)))
        off += w
    return np.concatenate(out, -1)


def groot_dense(t, m, n, tile_transpose=True):
    """GR00T's decode of a record (groot_tcq.py:143-191) in FP64."""
    seq = states_bit_by_bit(t['trellis'].view(torch.int16).numpy().view(np.uint16).reshape(-1, 32))
    s = seq.reshape(m // 16, n // 16, 16, 8)
    states = (s.transpose(0, 2, 1, 3) if tile_transpose else s.reshape(m // 16, 16, n // 16, 8)).reshape(m, n // 2)
    x = (states + 1) * states
    h = (x >> 6) & 511
    flip = 1 - 2 * ((x >> 15) & 1)
    k = np.stack([2 * h, 2 * h + 1], -1).reshape(m, n)
    sg = np.stack([flip, np.ones_like(flip)], -1).reshape(m, n)
    tl = t['tlut'].float().numpy().astype(np.float64)
    if tl.ndim == 3:
        G = tl.shape[0]
        q = tl.reshape(G, -1)[(np.arange(m) // (m // G))[:, None], k]
    else:
        q = tl.reshape(-1)[k]
    q = q * sg * t['row_scale'].float().numpy().astype(np.float64)[:, None]
    if t.get('col_scale') is not None:
        q = q * t['col_scale'].float().numpy().astype(np.float64)[None, :]
    if t.get('signs_out') is not None:
        q = (block_hadamard(q.T) * t['signs_out'].numpy().astype(np.float64)).T
    return block_hadamard(q) * t['signs'].numpy().astype(np.float64)


def oracle_of(tensors, name='l'):
    t = {k: (v.numpy() if torch.is_tensor(v) else v) for k, v in tensors.items()}
    return O.Layer(name, t)


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


CASES = [(1536, 512, False, True, 2), (512, 1536, True, False, 1), (256, 6144, True, True, 1), (1024, 1024, False, False, 4)]


@pytest.mark.parametrize('m,n,two_sided,col_scale,groups', CASES)
def test_groot_record_converts_to_the_same_weight(m, n, two_sided, col_scale, groups, tmp_path):
    rec = record(m, n, m + n, two_sided, col_scale, groups)
    path = tmp_path / 'layer.pt'
    torch.save(rec, path)
    t = F.from_groot(F._read_record(path))
    assert set(t) == {'bits', 'tlut', 'row_scale', 'su'} | ({'sv'} if two_sided else set()) | ({'col_scale'} if col_scale else set())
    assert t['bits'].dtype == torch.int16 and tuple(t['bits'].shape) == ((m // 16) * (n // 16), 32)
    ol = oracle_of(t)
    assert (ol.sv is None) == (not two_sided) and (ol.col_scale is None) == (not col_scale)
    want = groot_dense(rec['tensors'], m, n)
    assert rel(ol.dense('fp16'), want) < 1e-6
    # planted mistakes fail (swapped sign vectors: test_swapped_sign_vectors_fail)
    assert rel(groot_dense(rec['tensors'], m, n, tile_transpose=False), want) > 1e-2
    if col_scale:
        assert rel(oracle_of({k: v for k, v in t.items() if k != 'col_scale'}).dense('fp16'), want) > 1e-3


def test_swapped_sign_vectors_fail():
    """On a square two-sided layer, exchanging signs and signs_out changes the weight (the mapping is not symmetric)."""
    rec = record(512, 512, 3, True, False, 1)
    t = F.from_groot(rec)
    want = groot_dense(rec['tensors'], 512, 512)
    assert rel(oracle_of(t).dense('fp16'), want) < 1e-6
    assert rel(oracle_of(dict(t, su=t['sv'], sv=t['su'])).dense('fp16'), want) > 1e-2


def test_convert_groot_writes_the_deploy_schema(tmp_path):
    from safetensors.torch import load_file
    files = {}
    for i, case in enumerate(CASES):
        files[f'layer{i}'] = tmp_path / f'layer{i}.pt'
        torch.save(record(*case[:2], 50 + i, *case[2:]), files[f'layer{i}'])
    out = F.convert_groot(files, tmp_path / 'packed.safetensors')
    f = load_file(str(out))
    for i, (m, n, two_sided, col_scale, groups) in enumerate(CASES):
        rec = torch.load(files[f'layer{i}'], weights_only=True)['tensors']
        assert torch.equal(f[f'layer{i}::bits'], rec['trellis'].view(torch.int16).reshape(-1, 32))
        assert torch.equal(f[f'layer{i}::su'], rec['signs']) and torch.equal(f[f'layer{i}::tlut'], rec['tlut'])
        assert (f'layer{i}::sv' in f) == two_sided and (f'layer{i}::col_scale' in f) == col_scale


def test_records_outside_the_deploy_format_are_refused():
    rec = record(256, 256, 1, True, False, 1)
    with pytest.raises(ValueError):
        F.from_groot(dict(rec, tcq=dict(rec['tcq'], K=3)))
    bad = dict(rec['tensors'], trellis=rec['tensors']['trellis'][:-32])
    with pytest.raises(ValueError):
        F.from_groot(dict(tensors=bad))
    with pytest.raises(ValueError):
        F.from_groot(dict(tensors=dict(rec['tensors'], signs=rec['tensors']['signs'] * 0)))
