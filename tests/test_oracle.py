"""Pins the CPU oracle (oracle/tcq_oracle.py) to the reference's own arithmetic (golden vectors written by importing
deploy/tcq_kernels/tcq_format.py, tests/golden/make_golden.py) and to closed forms that do not share its code."""
import json

import numpy as np
import pytest

from oracle import tcq_oracle as O


def sylvester(n):
    H = np.ones((1, 1))
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def block_hadamard(n):
    """Dense FP64 normalised block Walsh matrix over the binary decomposition of n."""
    M, off = np.zeros((n, n)), 0
    for w in O.block_widths(n):
        M[off:off + w, off:off + w] = sylvester(w) / np.sqrt(w)
        off += w
    return M


def layer_from(golden, tag):
    t = {k: golden[f'{tag}_{k}'] for k in ('bits', 'tlut', 'row_scale', 'su', 'sv')}
    bias = golden[f'{tag}_bias'] if f'{tag}_bias' in golden.files else None
    return O.Layer(tag, t, bias=bias)


TAGS = ('l0', 'l1', 'l2', 'l3')


def test_block_widths(golden):
    ref = json.loads(str(golden['block_widths']))
    for w, b in ref.items():
        assert O.block_widths(int(w)) == b
        assert sum(b) == int(w) and all(x & (x - 1) == 0 for x in b) and b == sorted(b, reverse=True)


@pytest.mark.parametrize('w', [1, 2, 16, 48, 80, 256, 1152, 4304])
def test_fwht_golden_bitexact(golden, w):
    y = O.fwht(golden[f'fwht_x_{w}'])
    assert y.dtype == np.float32
    assert np.array_equal(y.view(np.uint32), golden[f'fwht_y_{w}'].view(np.uint32))


def test_fwht_signed_zero_and_ties(golden):
    y = O.fwht(golden['fwht_x_ties'])
    assert np.array_equal(y.view(np.uint32), golden['fwht_y_ties'].view(np.uint32))


@pytest.mark.parametrize('n', [1, 2, 8, 48, 1024, 1152, 4304])
def test_fwht_closed_form(n):
    x = np.random.default_rng(n).standard_normal((4, n)).astype(np.float32)
    y = O.fwht(x).astype(np.float64)
    ref = x.astype(np.float64) @ block_hadamard(n).T
    assert np.max(np.abs(y - ref)) < 1e-5 * max(1.0, np.abs(ref).max())
    # involution: the normalised transform is its own inverse
    assert np.allclose(O.fwht(O.fwht(x)), x, atol=1e-5)


def test_fwht_stage_order_matters():
    """The oracle's rounding is that of stage order h = 1, 2, 4, ...; the reverse order gives different bits on random data."""
    x = np.random.default_rng(3).standard_normal((8, 1024)).astype(np.float32) * 7
    y = O.fwht(x)
    z, h = x.copy(), 512
    while h >= 1:
        z = z.reshape(8, 1024 // (2 * h), 2, h)
        z = np.stack((z[:, :, 0] + z[:, :, 1], z[:, :, 0] - z[:, :, 1]), axis=2).reshape(8, 1024)
        h //= 2
    z = z * np.float32(1 / 32)
    assert np.allclose(y, z, atol=1e-4) and not np.array_equal(y, z)


def brute_states(bits, m, n):
    """Independent restatement: the 512-bit stream of each tile as a list of bits (MSB first), 16-bit windows at 4 t with
    wrap-around, tiles row-major, tile row r pair p -> state 8 r + p."""
    out = np.zeros((m, n // 2), dtype=np.int64)
    tiles_per_row = n // 16
    for tile in range(bits.shape[0]):
        I, J = divmod(tile, tiles_per_row)
        stream = []
        for wd in bits[tile].astype(np.uint16):
            stream += [(int(wd) >> (15 - k)) & 1 for k in range(16)]
        for t in range(128):
            v = 0
            for k in range(16):
                v = (v << 1) | stream[(4 * t + k) % 512]
            r, p = divmod(t, 8)
            out[16 * I + r, 8 * J + p] = v
    return out


@pytest.mark.parametrize('tag', TAGS)
def test_states_and_lookup_golden(golden, tag):
    L = layer_from(golden, tag)
    st = L.states()
    assert np.array_equal(st, golden[f'{tag}_states'].astype(np.int64))
    assert np.array_equal(O.lookup(st, L.tlut.astype(np.float32)).view(np.uint32), golden[f'{tag}_lookup_f32'].view(np.uint32))
    assert np.array_equal(L.t8, golden[f'{tag}_t8'])
    assert np.array_equal(L.rs.view(np.uint32), golden[f'{tag}_rs'].view(np.uint32))
    assert np.float32(L.gain).view(np.uint32) == golden[f'{tag}_gain'].view(np.uint32)
    assert np.array_equal(L.w8_reference(), golden[f'{tag}_w8'])


@pytest.mark.parametrize('tag', ('l0', 'l3'))
def test_states_brute_force(golden, tag):
    L = layer_from(golden, tag)
    assert np.array_equal(L.states(), brute_states(L.bits, L.m, L.n))


def test_state_recurrence():
    """Within a tile, s[t+1] = ((s[t] << 4) | nibble) & 0xffff and the stream is tail-biting: s[128] == s[0]."""
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 1 << 16, size=(4, 32), dtype=np.uint32).astype(np.uint16)
    st = O.states_from_bits(bits, 32, 32).reshape(2, 16, 2, 8).transpose(0, 2, 1, 3).reshape(4, 128)
    for tile in range(4):
        words = bits[tile].astype(np.int64)
        for t in range(128):
            nib = (words[((4 * t + 16) // 16) % 32] >> (12 - (4 * t + 16) % 16)) & 0xf
            assert st[tile, (t + 1) % 128] == ((st[tile, t] << 4) | nib) & 0xffff


def test_lookup_closed_form():
    rng = np.random.default_rng(11)
    table = rng.standard_normal((512, 2)).astype(np.float32)
    states = rng.integers(0, 1 << 16, size=(4, 6))
    v = O.lookup(states, table).reshape(4, 6, 2)
    for i in range(4):
        for j in range(6):
            s = int(states[i, j]); x = (s + 1) * s
            h = (x >> 6) % 512
            sign = -1.0 if (x >> 15) & 1 else 1.0
            assert v[i, j, 0] == sign * table[h, 0] and v[i, j, 1] == table[h, 1]


@pytest.mark.parametrize('tag', ('snap_neg', 'snap_tiny'))
def test_snap_golden(golden, tag):
    t8, rs, g = O.snap(golden[f'{tag}_tlut'], golden[f'{tag}_row_scale'])
    assert np.array_equal(t8, golden[f'{tag}_t8'])
    assert np.array_equal(rs.view(np.uint32), golden[f'{tag}_rs'].view(np.uint32))
    assert np.float32(g).view(np.uint32) == golden[f'{tag}_gain'].view(np.uint32)
    assert np.abs(t8).max() == 127


def test_snap_gain_is_reciprocal_multiply():
    """The gain is float32(1/amax) * 127, not 127 / amax: on many tables the two differ in the last bit."""
    rng = np.random.default_rng(5)
    diff = 0
    for _ in range(400):
        amax = np.float32(rng.uniform(1.0, 5.0))
        a = np.float32(np.float32(1.0) / amax) * np.float32(127.0)
        b = np.float32(127.0) / amax
        diff += a != b
        tl = np.zeros((512, 2), np.float16); tl[0, 0] = amax
        assert O.snap(tl, np.ones(16, np.float16))[2] == np.float32(np.float32(1.0) / np.float32(np.float16(amax))) * np.float32(127)
    assert diff > 0


def test_quantize_tokens_golden(golden):
    q, s = O.quantize_tokens(golden['qt_h'])
    assert np.array_equal(q, golden['qt_q'])
    assert np.array_equal(s.view(np.uint32), golden['qt_s'].view(np.uint32))
    assert s[2, 0] == 1.0 and not q[2].any()


def test_quantize_tokens_closed_form():
    h = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -127.0, 63.5]], np.float32)
    q, s = O.quantize_tokens(h)
    assert s[0, 0] == 1.0
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -127, 64]]        # half-way cases round to even


def test_int_matmul(golden):
    acc = O.int_matmul(golden['im_a'], golden['im_b'])
    assert np.array_equal(acc, golden['im_acc'])
    brute = golden['im_a'].astype(np.int64) @ golden['im_b'].astype(np.int64).T
    assert np.array_equal(acc, brute.astype(np.int32))


@pytest.mark.parametrize('tag', TAGS)
def test_dense_golden_and_closed_form(golden, tag):
    L = layer_from(golden, tag)
    for table in ('fp16', 'int8'):
        d = L.dense(table)
        assert np.array_equal(d.view(np.uint32), golden[f'{tag}_dense_{table}'].view(np.uint32))
    q = O.lookup(L.states(), L.tlut.astype(np.float32)).astype(np.float64) * L.row_scale.astype(np.float64)[:, None]
    W = np.diag(L.sv.astype(np.float64)) @ block_hadamard(L.m) @ q @ block_hadamard(L.n) @ np.diag(L.su.astype(np.float64))
    assert np.allclose(L.dense('fp16'), W, atol=1e-5)


@pytest.mark.parametrize('tag', TAGS)
@pytest.mark.parametrize('dt', ('f32', 'bf16'))
def test_reference_linear_golden(golden, tag, dt):
    L = layer_from(golden, tag)
    x = golden[f'{tag}_x_{dt}']
    x = O.bf16_to_f32(x) if dt == 'bf16' else x
    for a8 in ('a8', 'a16'):
        for table in ('int8', 'fp16'):
            y = O.reference_linear(x, L, a8=a8 == 'a8', table=table)
            yf = O.reference_linear(x, L, a8=a8 == 'a8', table=table, out_dtype='f32')
            gy = golden[f'{tag}_y_{dt}_{a8}_{table}'].view(np.uint16)
            gyf = golden[f'{tag}_yf_{dt}_{a8}_{table}']
            if a8 == 'a8' and table == 'int8':
                assert np.array_equal(y, gy) and np.array_equal(yf.view(np.uint32), gyf.view(np.uint32))
            else:      # FP64 matmul: summation order of the BLAS differs from PyTorch's
                assert np.allclose(yf, gyf, rtol=1e-6, atol=1e-6)
                assert np.max(np.abs(y.astype(np.int32) - gy.astype(np.int32))) <= 1


@pytest.mark.parametrize('tag', TAGS)
def test_reference_linear_matches_dense_weight(golden, tag):
    """a8=False, FP16 table: y = x W^T with W = S_v H_m diag(r) Q H_n S_u (FP64 closed form)."""
    L = layer_from(golden, tag)
    x = golden[f'{tag}_x_f32']
    y = O.reference_linear(x, L, a8=False, table='fp16', out_dtype='f32')
    ref = x.astype(np.float64) @ L.dense('fp16').astype(np.float64).T
    if L.bias is not None:
        ref = ref + L.bias
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6


def test_gelu_matches_reference_table(golden):
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(O.gelu_tanh_bf16(allb), golden['gelu_bf16_all'].view(np.uint16))


def test_bf16_rounding():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, np.nan, -0.0, np.inf], np.float32)
    b = O.bf16_bits(x)
    assert b.tolist() == [0x3f80, 0x3f80, 0x3f82, 0x3f80, 0x7fc0, 0x8000, 0x7f80]


def test_mlp_middle_is_the_unfused_chain():
    rng = np.random.default_rng(2)
    N = 64
    zg, zu = rng.standard_normal((3, N)).astype(np.float32), rng.standard_normal((3, N)).astype(np.float32)
    svg, svu, su = [np.where(rng.integers(0, 2, N) > 0, 1, -1).astype(np.int8) for _ in range(3)]
    q, s, g, u = O.mlp_middle(zg, zu, svg, svu, su)
    yg = O.bf16_to_f32(O.bf16_bits(O.fwht(zg) * svg.astype(np.float32)))
    import torch
    act = torch.nn.functional.gelu(torch.from_numpy(yg).bfloat16(), approximate='tanh')
    yu = torch.from_numpy(O.bf16_to_f32(O.bf16_bits(O.fwht(zu) * svu.astype(np.float32)))).bfloat16()
    prod = (act * yu).float().numpy()
    q2, s2 = O.quantize_tokens(O.fwht(prod * su.astype(np.float32)))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_plain_middle_is_the_unfused_chain():
    """mid1's definition through PyTorch's own BF16 cast and GELU; the bias enters before the BF16 rounding."""
    import torch
    rng = np.random.default_rng(3)
    N = 96                                                   # 64 + 32: two Walsh blocks
    z = rng.standard_normal((4, N)).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.3).astype(np.float32)
    sv, su = [np.where(rng.integers(0, 2, N) > 0, 1, -1).astype(np.int8) for _ in range(2)]
    q, s, g = O.plain_middle(z, sv, bias, su)
    y = torch.from_numpy(O.fwht(z) * sv.astype(np.float32) + bias).bfloat16()
    act = torch.nn.functional.gelu(y, approximate='tanh').float().numpy()
    assert np.array_equal(g, torch.from_numpy(act).bfloat16().view(torch.int16).numpy().astype(np.uint16))
    q2, s2 = O.quantize_tokens(O.fwht(act * su.astype(np.float32)))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    qb, _, _ = O.plain_middle(z, sv, None, su)               # the bias matters
    assert not np.array_equal(q, qb)


def test_q4_layout():
    q = np.arange(2 * 8, dtype=np.int8).reshape(2, 8)
    q4 = O.q4_layout(q)
    assert q4.shape == (2, 2)
    assert q4[1, 0] == int.from_bytes(bytes([4, 5, 6, 7]), 'little')
    assert q4[0, 1] == int.from_bytes(bytes([8, 9, 10, 11]), 'little')


def test_rmsnorm_close_to_the_formula():
    """The kernels' RMSNorm (fixed summation order) against the Gemma formula in FP64: at most one BF16 rounding apart, and
    a wrong term (no +1 on the weight, mean over K-1, eps dropped) moves it far."""
    rng = np.random.default_rng(4)
    M, K = 6, 1024
    x = O.bf16_to_f32(O.bf16_bits(rng.standard_normal((M, K)).astype(np.float32) * 3))
    x[5] *= 1e-4                                              # eps matters for this row
    w = O.bf16_bits(rng.standard_normal(K).astype(np.float32) * 0.1)
    eps = 1e-6
    y = O.bf16_to_f32(O.rmsnorm_bf16(x, w, eps)).astype(np.float64)
    x64, w64 = x.astype(np.float64), O.bf16_to_f32(w).astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + eps) * (1 + w64)
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30)
    bad = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + eps) * w64
    assert np.abs(y - bad).max() > 0.1
    bad_eps = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True)) * (1 + w64)
    assert np.abs(y[5] - bad_eps[5]).max() > 1e-3 * np.abs(bad_eps[5]).max()


def test_row_group_tables():
    """(G, 512, 2) row-group tables: G = 1 is the single table; each group's rows equal the single-table path on that group's
    rows and table (groot_tcq.py decode_normalized), and each table snaps on its own."""
    rng = np.random.default_rng(12)
    m, n, G = 64, 32, 4
    bits = rng.integers(0, 1 << 16, size=((m // 16) * (n // 16), 32), dtype=np.uint32).astype(np.uint16).view(np.int16)
    tabs = rng.standard_normal((G, 512, 2)).astype(np.float32) * np.arange(1, G + 1)[:, None, None]
    st = O.states_from_bits(bits, m, n)
    assert np.array_equal(O.lookup(st, tabs[:1]), O.lookup(st, tabs[0]))
    got = O.lookup(st, tabs)
    rpg = m // G
    for g in range(G):
        assert np.array_equal(got[g * rpg:(g + 1) * rpg], O.lookup(st[g * rpg:(g + 1) * rpg], tabs[g]))
    rsc = rng.uniform(0.5, 1.5, m).astype(np.float16)
    t8, rs, gain = O.snap(tabs.astype(np.float16), rsc)
    assert t8.shape == (G, 512, 2) and gain.shape == (G,)
    for g in range(G):
        t8g, rsg, gg = O.snap(tabs[g].astype(np.float16), rsc[g * rpg:(g + 1) * rpg])
        assert np.array_equal(t8[g], t8g) and np.array_equal(rs[g * rpg:(g + 1) * rpg], rsg) and gain[g] == gg
    assert len(set(gain.tolist())) == G                                   # the tables really differ


# ------------------------------------------------------------------------------- W2 float path (Group.run_float)
def _w2i(golden):
    t = {k: golden[f'w2i_{k}'] for k in ('bits', 'tlut', 'row_scale', 'su', 'sv')}
    return O.Layer('w2i', t, bias=golden['w2i_bias'])


def _bf16_torch(a):
    """BF16 rounding by PyTorch's own cast (the library routine), back to float32."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def test_w2_inputs_rotate_to_exact_integers(golden):
    L = _w2i(golden)
    v = golden['w2i_v']
    assert np.array_equal(O.fwht(golden['w2i_x'] * L.su.astype(np.float32)), v)
    assert np.array_equal(O.fwht(golden['w2i_xb'] * L.su.astype(np.float32)), v + np.float32(1 / 32))
    assert np.array_equal(L.w8_reference(), golden['w2i_w8'])


def test_w2_linear_expert_equals_reference_on_bf16_exact_activations(golden):
    """Expert variant (deploy/tcq_kernels/modules.py:131-142): with rotated activations that BF16 holds exactly, the W2 float
    path is the reference's a8=False layer (tcq_format.py:137-138) bit for bit; with activations v + 1/32 its BF16 rounding
    of h brings them back to v. Leaving the rounding out, or rounding the accumulator, fails."""
    L = _w2i(golden)
    ref = golden['w2i_y_bf16'].view(np.uint16)
    assert np.array_equal(O.w2_linear(golden['w2i_x'], L, small=True), ref)
    assert np.array_equal(O.w2_linear(golden['w2i_xb'], L, small=True), ref)
    # planted slips: h not rounded (the reference's own a8=False layer on x_b), accumulator rounded as well
    assert not np.array_equal(O.reference_linear(golden['w2i_xb'], L, a8=False, table='int8'), ref)
    assert not np.array_equal(O.w2_linear(golden['w2i_x'], L, small=False), ref)


def test_w2_linear_prefill_rounds_the_accumulator(golden):
    """Prefill variant (modules.py:120-130): h @ W.t() in BF16 -> the FP32 sum rounded to BF16, then k_post_bf16 scales it by
    rs (SCALE = bf2f(a) * rs, kernels.py:545). Expected value from the exact integer product, PyTorch's BF16 cast, and the
    golden-pinned output rotation; slips (no rounding, rounding after the row scale) fail."""
    L = _w2i(golden)
    v = golden['w2i_v'].astype(np.int64)
    acc = (v @ golden['w2i_w8'].astype(np.int64).T).astype(np.float32)     # exact: |acc| < 2^24
    assert np.abs(acc).max() < 2 ** 24

    def post(z):
        y = O.fwht(z) * L.sv.astype(np.float32) + golden['w2i_bias']
        return _bf16_torch_bits(y)

    want = post(_bf16_torch(acc) * L.rs[None, :])
    got = O.w2_linear(golden['w2i_x'], L, small=False)
    assert np.array_equal(got, want)
    assert np.array_equal(O.w2_linear(golden['w2i_xb'], L, small=False), want)
    assert not np.array_equal(post(acc * L.rs[None, :]), want)                    # no accumulator rounding
    assert not np.array_equal(post(_bf16_torch(acc * L.rs[None, :])), want)       # rounding after the row scale
    # the unrounded post equals the golden reference output, so `post` is the reference's output half
    assert np.array_equal(post(acc * L.rs[None, :]), golden['w2i_y_bf16'].view(np.uint16))


def _bf16_torch_bits(y):
    import torch
    return torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------- GR00T records: one-sided layers, column scales
@pytest.mark.parametrize('m,n,one_sided,cs', [(64, 1536, True, True), (48, 96, True, False), (96, 64, False, True),
                                              (32, 3072, True, True), (48, 48, False, False)])
def test_groot_layer_forms_against_the_dense_closed_form(m, n, one_sided, cs):
    """Layer.dense and reference_linear (FP16 table, unquantized activations) equal the FP64 closed form
    W = [S_v H_m] diag(r) Q diag(c) H_n S_u (groot_tcq.py:178-191) built from explicit Sylvester blocks; putting c on the
    output side, leaving it out, or rotating the output of a one-sided layer fails."""
    L = O.random_layer(m, n, 7 * m + n, bias=True, per_layer_scale=False, one_sided=one_sided, col_scale=cs)
    Q = O.lookup(L.states(), L.tlut.astype(np.float32)).astype(np.float64)
    r = L.row_scale.astype(np.float64)
    c = L.col_scale.astype(np.float64) if cs else np.ones(n)
    W = ((r[:, None] * Q * c[None, :]) @ block_hadamard(n).T) * L.su.astype(np.float64)[None, :]
    if not one_sided:
        W = L.sv.astype(np.float64)[:, None] * (block_hadamard(m) @ W)
    scale = np.abs(W).max()
    assert np.max(np.abs(L.dense('fp16') - W)) < 1e-5 * scale
    x = np.random.default_rng(n).standard_normal((5, n)).astype(np.float32)
    y = O.reference_linear(x, L, a8=False, table='fp16', out_dtype='f32').astype(np.float64)
    want = x.astype(np.float64) @ W.T + L.bias
    assert np.max(np.abs(y - want)) < 1e-4 * np.abs(want).max()
    # planted slips
    if cs:
        W_noc = ((r[:, None] * Q) @ block_hadamard(n).T) * L.su.astype(np.float64)[None, :]
        if not one_sided:
            W_noc = L.sv.astype(np.float64)[:, None] * (block_hadamard(m) @ W_noc)
        assert np.max(np.abs(x @ W_noc.T + L.bias - want)) > 1e-2 * np.abs(want).max()      # c left out
    if one_sided:
        rotated = O.fwht(np.ascontiguousarray((x.astype(np.float64) @ W.T).astype(np.float32))) + L.bias
        assert np.max(np.abs(rotated - want)) > 1e-2 * np.abs(want).max()
    # the W2A8 path quantizes the column-scaled rotated activations: within the INT8 rounding of the closed form
    yq = O.reference_linear(x, L, a8=True, table='fp16', out_dtype='f32').astype(np.float64)
    assert np.linalg.norm(yq - want) < 2e-2 * np.linalg.norm(want)


def test_groot_one_sided_int8_layer_is_the_scaled_product():
    """One-sided W2A8 layer: y = bf16((acc * s) * rs + bias), acc = int_matmul(quantize_tokens(fwht(x * su) * c), w8) exact
    (tcq_format.py:130-136 without the output rotation, groot_tcq.py:187-191)."""
    L = O.random_layer(64, 1536, 11, bias=True, one_sided=True, col_scale=True)
    x = np.random.default_rng(3).standard_normal((4, 1536)).astype(np.float32)
    h = O.fwht(x * L.su.astype(np.float32)) * L.col_scale.astype(np.float32)
    q, s = O.quantize_tokens(h)
    acc = (q.astype(np.int64) @ L.w8_reference().astype(np.int64).T).astype(np.int32)
    want = O.bf16_bits((acc.astype(np.float32) * s) * L.rs[None, :] + L.bias)
    assert np.array_equal(O.reference_linear(x, L), want)
