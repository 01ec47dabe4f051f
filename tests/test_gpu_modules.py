"""GPU tests of the module layer: Layer / load, RefLinear and the grouped KLinear / KGatedMLP path against the oracle,
the operating points against each other, install on a Gemma-shaped expert, and HIP-graph replays of an action chunk."""
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
    """The oracle twin of a device Layer (same packed tensors)."""
    t = dict(bits=L.bits.cpu().numpy(), tlut=L.tlut.cpu().numpy(), row_scale=L.row_scale.cpu().numpy(),
             su=L.su.cpu().numpy(), sv=L.sv.cpu().numpy())
    return O.Layer(L.name, t, bias=None if L.bias is None else L.bias.cpu().numpy())


def device_layer(m, n, seed, bias=False, name='layer', groups=1):
    from yanlongvla_amd import tcq_format as F
    ol = O.random_layer(m, n, seed, name=name, bias=bias, per_layer_scale=False, groups=groups)
    t = dict(bits=torch.from_numpy(ol.bits), tlut=torch.from_numpy(ol.tlut), row_scale=torch.from_numpy(ol.row_scale),
             su=torch.from_numpy(ol.su), sv=torch.from_numpy(ol.sv))
    return F.Layer(name, t, bias=None if ol.bias is None else torch.from_numpy(ol.bias), device=DEV), ol


def bits16(y):
    return y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def differ(a, b):
    """Where two bit arrays differ: count, first positions, their values (for the assertion message)."""
    d = np.argwhere(a != b)
    return f'{len(d)} of {a.size} differ; first {d[:6].tolist()}: {a[tuple(d[:6].T)].tolist()} vs {b[tuple(d[:6].T)].tolist()}'


def test_layer_derived_tensors_and_dense():
    L, ol = device_layer(256, 1024, 3)
    assert np.array_equal(L.t8.cpu().numpy(), ol.t8)
    assert np.array_equal(L.rs.cpu().numpy().view(np.uint32), ol.rs.view(np.uint32))
    assert np.array_equal(L.w8_reference().cpu().numpy(), ol.w8_reference())
    for table in ('fp16', 'int8'):
        assert np.array_equal(L.dense(table).cpu().numpy(), ol.dense(table))


@pytest.mark.parametrize('M', [1, 50, 130])
@pytest.mark.parametrize('bias', [False, True])
def test_reflinear_bitexact(M, bias):
    from yanlongvla_amd.modules import RefLinear
    L, ol = device_layer(512, 1024, 10 + M, bias=bias)
    x = torch.randn(M, 1024, device=DEV).bfloat16()
    ref = O.reference_linear(x.float().cpu().numpy(), ol)
    for resident in (True, False):
        y = RefLinear(L, resident=resident)(x)
        assert y.dtype == torch.bfloat16 and np.array_equal(bits16(y), ref)


@pytest.mark.parametrize('table', ['int8', 'fp16'])
def test_reflinear_float_activations(table):
    from yanlongvla_amd.modules import RefLinear
    L, ol = device_layer(256, 512, 21)
    x = torch.randn(7, 512, device=DEV)
    ref = O.reference_linear(x.cpu().numpy(), ol, a8=False, table=table, out_dtype='f32')
    y = RefLinear(L, a8=False, table=table)(x).float().cpu().numpy()
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 4e-3            # BF16 output of an FP32 result


def test_reflinear_int8_activations_fp16_table():
    """a8 with the FP16 table (tcq_format.py:139-141): INT8 activations and scales bit-exact, FP64 sums on both sides in
    their own orders, so the BF16 outputs agree to within one BF16 rounding of a few elements."""
    from yanlongvla_amd.modules import RefLinear
    L, ol = device_layer(256, 512, 22)
    x = torch.randn(9, 512, device=DEV).bfloat16()
    ref = O.reference_linear(x.float().cpu().numpy(), ol, a8=True, table='fp16')
    y = bits16(RefLinear(L, a8=True, table='fp16')(x))
    close = O.bf16_to_f32(ref)
    assert np.mean(y == ref) > 0.99
    assert np.linalg.norm(O.bf16_to_f32(y) - close) / np.linalg.norm(close) < 2e-3


def qkv_layers(seed, K=1024, widths=(2048, 256, 256), bias=False):
    from yanlongvla_amd import tcq_format as F
    layers, oracles = [], []
    su = None
    for i, m in enumerate(widths):
        L, ol = device_layer(m, K, seed + i, bias=bias, name=f'p.layers.0.self_attn.{("q", "k", "v")[i]}_proj')
        if su is None:
            su = L.su
        L.su = su
        ol.su = su.cpu().numpy()
        layers.append(L)
        oracles.append(ol)
    return layers, oracles


@pytest.mark.parametrize('M', [1, 50, 64, 65, 300])
@pytest.mark.parametrize('mode', ['fly', 'resident', 'chunk'])
def test_group_bitexact(M, mode):
    """q / k / v group: one rotation + quantization, one product (small-M kernels up to 64 tokens, INT8 MFMA GEMM above),
    one batched epilogue; every member's BF16 output equals the oracle's layer bit for bit."""
    from yanlongvla_amd.modules import Group, KLinear
    layers, oracles = qkv_layers(100 + M, bias=M == 50)
    g = Group(layers, 'expert' if M <= 64 else 'llm', mode)
    mods = [KLinear(g, i) for i in range(3)]
    x = torch.randn(M, 1024, device=DEV).bfloat16()
    xs = x.float().cpu().numpy()
    for mod, ol in zip(mods, oracles):
        y = mod(x)
        assert np.array_equal(bits16(y), O.reference_linear(xs, ol))
    assert g.pending is None                                        # all three members served


@pytest.mark.parametrize('M', [10, 50, 200])
@pytest.mark.parametrize('split', [False, True])
def test_gated_mlp_bitexact(M, split):
    """KGatedMLP (fused middle) == the unfused chain: gate / up layers, BF16 GELU(gate) * up, down layer. GELU is the
    device table both sides (PyTorch's GELU on the GPU, as the reference tabulates it, kernels.py:563-569): PyTorch's CPU
    GELU differs from it in the last bit for some BF16 inputs, so a gate value on such an input would differ by design."""
    from yanlongvla_amd import kernels as K, modules
    from yanlongvla_amd.modules import Group, KGatedMLP
    gate, og = device_layer(4096, 1024, 7, name='p.mlp.gate_proj')
    up, ou = device_layer(4096, 1024, 8, name='p.mlp.up_proj')
    up.su = gate.su
    ou.su = og.su
    down, od = device_layer(1024, 4096, 9, name='p.mlp.down_proj')
    old = modules.FUSE['split']
    modules.FUSE['split'] = split
    try:
        mlp = KGatedMLP(Group([gate, up], 'expert', 'fly'), Group([down], 'expert', 'fly'))
        x = torch.randn(M, 1024, device=DEV).bfloat16()
        y = mlp(x)
    finally:
        modules.FUSE['split'] = old
    xs = x.float().cpu().numpy()
    gb = O.reference_linear(xs, og)
    ub = O.reference_linear(xs, ou)
    lut = K.gelu_table(DEV).view(torch.int16).cpu().numpy().view(np.uint16)
    prod = O.bf16_bits(O.bf16_to_f32(lut[gb]) * O.bf16_to_f32(ub))
    ref = O.reference_linear(O.bf16_to_f32(prod), od)
    assert np.array_equal(bits16(y), ref), differ(bits16(y), ref)


def small_expert(layers=2, prefix=64, seed=0):
    from yanlongvla_amd import gemma
    model = gemma.make_policy(gemma.ExpertPolicy, DEV, seed=seed, layers=layers)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    ks = [torch.randn(prefix, 256, generator=g, device=DEV).bfloat16() for _ in range(layers)]
    vs = [torch.randn(prefix, 256, generator=g, device=DEV).bfloat16() for _ in range(layers)]
    model.set_prefix(ks, vs)
    return model


def test_install_operating_points_agree():
    """The fused groups (fly / resident / hybrid) give the same action chunk as RefLinear layer by layer, bit for bit."""
    from yanlongvla_amd import gemma, modules
    outs, infos = {}, {}
    noise = torch.randn(50, 32, generator=torch.Generator(device=DEV).manual_seed(5), device=DEV)
    for runtime in ('reference', 'fly', 'resident', 'hybrid'):
        model = small_expert()
        layers = gemma.synthetic_layers(model, 11, DEV)
        infos[runtime] = modules.install(model, runtime=runtime, layers=layers)
        if runtime == 'hybrid':
            assert modules.decode_chunk(model) == 14
        outs[runtime] = model.sample_chunk(noise, steps=3)
    assert infos['fly']['groups'] == 2 * 4 and infos['fly']['fused_mlps'] == 2
    assert infos['hybrid']['modes'] == {'resident': 0, 'fly': 0, 'chunk': 8}
    for r in ('fly', 'resident', 'hybrid'):
        assert torch.equal(outs[r], outs['reference']), r
    assert torch.isfinite(outs['fly']).all()


@pytest.mark.parametrize('part', ['expert', 'backbone'])
def test_chained_prologues_bitexact(part):
    """A decoder layer's last epilogue computing the next layer's norm + rotate + quantize prologue (FUSE['chain']) gives
    the same outputs as each layer running its own tcq_norm_pre, and the hand-off is taken at every layer boundary: a
    3-layer expert over a 2-step chunk (inside inference mode), and a 3-layer backbone over a 120-token prefill plus 2
    decode steps (version counters)."""
    from yanlongvla_amd import gemma, modules
    outs, taken = {}, {}
    for chain in (False, True):
        modules.FUSE['chain'] = chain
        try:
            if part == 'expert':
                model = small_expert(layers=3, seed=4)
                modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, 13, DEV))
                noise = torch.randn(50, 32, generator=torch.Generator(device=DEV).manual_seed(6), device=DEV)
                before = modules.STATS['chained_prologues'] + modules.STATS['deferred_outputs']
                with torch.inference_mode():                 # inference tensors: the identity check
                    outs[chain] = [model.sample_chunk(noise, steps=2)]
                expect = 2 * 2
            else:
                model = gemma.make_policy(gemma.BackbonePolicy, DEV, seed=5, layers=3, vocab=512)
                modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, 14, DEV))
                x = torch.randn(120, 2048, generator=torch.Generator(device=DEV).manual_seed(7), device=DEV).bfloat16()
                before = modules.STATS['chained_prologues'] + modules.STATS['deferred_outputs']
                h, ks, vs = model.prefill(x)
                outs[chain] = [h]
                for t in range(2):
                    h, ks, vs = model.decode_step(x[t:t + 1], ks, vs)
                    outs[chain].append(h)
                expect = 2 * 3                               # decode steps: deferred outputs, counted alike
            taken[chain] = modules.STATS['chained_prologues'] + modules.STATS['deferred_outputs'] - before
        finally:
            modules.FUSE['chain'] = True
    assert taken == {False: 0, True: expect}
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)


@pytest.mark.parametrize('runtime', ['fly', 'resident'])
@pytest.mark.parametrize('flag,stat', [('prologue', 'layer_prologues'), ('pre_prologue', 'pre_prologues'),
                                       ('defer', 'deferred_outputs'), ('attn_prologue', 'attn_prologues'),
                                       ('attn_post', 'attn_posts')])
def test_prologues_in_the_mlp_products_bitexact(runtime, flag, stat):
    """At one token the o epilogue + residual + norm2 + rotate + quantize run inside the gate | up product's launch
    (FUSE['prologue']), the down projection's rotate + quantize inside the down product's (FUSE['pre_prologue']), and,
    in the decode loop, a layer's down epilogue + residual + the next layer's norm1 prologue inside the next q/k/v
    product's (FUSE['defer']), and the attention's chunk merge + o rotate + quantize inside the o product's
    (FUSE['attn_prologue']), with the q/k/v epilogue inside the attention's (FUSE['attn_post']): a 3-layer backbone's
    decode steps give the hidden states and key / value rows of the separate
    launches bit for bit. The MLP forms are taken at every layer of every step on the fly runtime's spread middle (the
    resident runtime keeps the separate launches); the deferred output at every layer boundary and the attention forms at
    every layer of both runtimes."""
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.BackbonePolicy, DEV, seed=5, layers=3, vocab=512)
    modules.install(model, runtime=runtime, layers=gemma.synthetic_layers(model, 15, DEV))
    x = torch.randn(60, 2048, generator=torch.Generator(device=DEV).manual_seed(9), device=DEV).bfloat16()
    _, ks, vs = model.prefill(x)
    outs, taken = {}, {}
    for fuse in (False, True):
        modules.FUSE[flag] = fuse
        try:
            before = modules.STATS[stat]
            k2, v2, outs[fuse] = ks, vs, []
            for t in range(2):
                h, k2, v2 = model.decode_step(x[t:t + 1], k2, v2)
                outs[fuse] += [h] + list(k2) + list(v2)
            taken[fuse] = modules.STATS[stat] - before
        finally:
            modules.FUSE[flag] = True
    expect = 2 * 2 if flag == 'defer' else 2 * 3 if (flag in ('attn_prologue', 'attn_post') or runtime == 'fly') else 0
    assert taken == {False: 0, True: expect}
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a, b)


def test_deferred_output_completed_when_the_next_layer_takes_another_input():
    """Inside deferred_outputs() a layer returns its output row uncomputed; when the next layer is called on a different
    tensor, it writes that row first (as tcq_post_add_norm_pre would have), so the returned output holds the same bits as
    without deferral, and the next layer runs its own norm prologue."""
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.BackbonePolicy, DEV, seed=6, layers=2, vocab=512)
    modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, 16, DEV))
    g = torch.Generator(device=DEV).manual_seed(10)
    x = torch.randn(40, 2048, generator=g, device=DEV).bfloat16()
    _, ks, vs = model.prefill(x)
    L0, L1 = model.stack.layers[0], model.stack.layers[1]
    tok, other = x[5:6].clone(), torch.randn(1, 2048, generator=g, device=DEV).bfloat16()
    ref0 = L0(tok, ks[0], vs[0])[0].clone()
    ref1 = L1(other, ks[1], vs[1])[0].clone()
    before = modules.STATS['deferred_outputs']
    with modules.deferred_outputs():
        out0 = L0(tok, ks[0], vs[0])[0]
        out1 = L1(other, ks[1], vs[1])[0]
    assert modules.STATS['deferred_outputs'] == before
    assert torch.equal(out0, ref0) and torch.equal(out1, ref1)


@pytest.mark.parametrize('runtime', ['reference', 'fly', 'resident'])
def test_kv_cache_decode_matches_concatenation(runtime):
    """Decode steps on a KVCache (the new rows written in place: by the q/k/v epilogue on the fused layers, by a copy on
    the reference runtime's) give the hidden states and key / value rows of decode_step's concatenated caches bit for bit;
    a rewound cache replays the same steps, and a full cache refuses another row."""
    from yanlongvla_amd import gemma, modules
    model = gemma.make_policy(gemma.BackbonePolicy, DEV, seed=5, layers=2, vocab=512)
    modules.install(model, runtime=runtime, layers=gemma.synthetic_layers(model, 14, DEV))
    x = torch.randn(70, 2048, generator=torch.Generator(device=DEV).manual_seed(8), device=DEV).bfloat16()
    with torch.inference_mode():
        _, ks, vs = model.prefill(x)
        cache = gemma.KVCache(ks, vs, 3)
        ref = []
        for t in range(3):
            h, ks, vs = model.decode_step(x[t:t + 1], ks, vs)
            ref.append(h)
        for _ in range(2):
            cache.rewind()
            got = [model.decode_step_cached(x[t:t + 1], cache) for t in range(3)]
            assert all(torch.equal(a, b) for a, b in zip(got, ref))
            assert cache.length == 73
            for i in range(2):
                assert torch.equal(cache.k[i], ks[i]) and torch.equal(cache.v[i], vs[i])
        with pytest.raises(RuntimeError):
            model.decode_step_cached(x[:1], cache)


def test_load_from_packed_file(tmp_path):
    from yanlongvla_amd import gemma, modules
    from yanlongvla_amd import tcq_format as F
    model = small_expert(layers=1)
    layers = gemma.synthetic_layers(model, 3, DEV)
    p = F.save({n: dict(bits=L.bits, tlut=L.tlut, row_scale=L.row_scale, su=L.su, sv=L.sv) for n, L in layers.items()},
               tmp_path / 'packed.safetensors')
    info = modules.install(model, row=p, runtime='fly')
    assert info['layers'] == 7 and info['fused_mlps'] == 1
    x = torch.randn(50, 32, device=DEV)
    twin = small_expert(layers=1)
    modules.install(twin, runtime='fly', layers=layers)
    assert torch.equal(model.velocity(x), twin.velocity(x))


def test_chunk_graph_replays_match_eager():
    """A captured action chunk (fused groups, small-M kernels, by-value descriptors) replays to the eager result, several
    times, with eager work in between."""
    from yanlongvla_amd import gemma, modules
    model = small_expert()
    modules.install(model, runtime='fly', layers=gemma.synthetic_layers(model, 2, DEV))
    noise = torch.randn(50, 32, device=DEV)
    eager = model.sample_chunk(noise, steps=2)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model.sample_chunk(noise, steps=2)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = model.sample_chunk(noise, steps=2)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(model.sample_chunk(noise, steps=2), eager)


def test_chunk_close_to_cpu_oracle():
    """One flow step of a 2-layer expert against the same model on the CPU with every quantized Linear computed by the
    oracle's reference_linear: the quantized layers are bit-exact on equal inputs, the PyTorch ops between them (norms,
    attention) round differently on CPU and GPU, so the velocity is compared in relative L2."""
    from yanlongvla_amd import gemma, modules
    model = small_expert()
    layers = gemma.synthetic_layers(model, 4, DEV)
    oracles = {n: oracle_of(L) for n, L in layers.items()}
    cpu = gemma.ExpertPolicy(layers=2).bfloat16().requires_grad_(False)
    cpu.load_state_dict({k: v.cpu() for k, v in model.state_dict().items()}, strict=False)
    cpu.set_prefix([k.cpu() for k in model.prefix_k], [v.cpu() for v in model.prefix_v])

    class OracleLinear(torch.nn.Module):
        def __init__(self, ol):
            super().__init__()
            self.ol, self.w8 = ol, ol.w8_reference()

        def forward(self, x):
            y = O.reference_linear(x.float().reshape(-1, self.ol.n).numpy(), self.ol, w8=self.w8)
            return torch.from_numpy(y.view(np.int16)).view(torch.bfloat16).reshape(*x.shape[:-1], self.ol.m)

    for n, ol in oracles.items():
        modules.set_submodule(cpu, n, OracleLinear(ol))
    modules.install(model, runtime='fly', layers=layers)
    x = torch.randn(50, 32)
    v_gpu = model.velocity(x.to(DEV)).float().cpu()
    v_cpu = cpu.velocity(x).float()
    assert (v_gpu - v_cpu).norm() / v_cpu.norm() < 2e-2


# ---------------------------------------------------------------------------------------------------- W2 float path
def test_decode_bf16_bitexact():
    """BF16 decode == the INT8 decode's values; the sign flips bit 15 as in k_decode_bf16 (kernels.py:320-337), so a zero
    table value with the sign bit set decodes to -0.0 (bit-exact after mapping -0.0 -> +0.0)."""
    from yanlongvla_amd import kernels as K
    L, ol = device_layer(256, 512, 31)
    tb = L.t8.to(torch.bfloat16).contiguous()
    out = torch.empty(256, 512, dtype=torch.bfloat16, device=DEV)
    K.decode_bf16(L.bits, tb, out)
    got = bits16(out)
    got = np.where(got == 0x8000, 0, got).astype(np.uint16)
    assert np.array_equal(got, O.bf16_bits(ol.w8_reference().astype(np.float32)))


@pytest.mark.parametrize('M,N,K', [(800, 2048, 1024), (65, 4096, 1024), (1, 1024, 4096), (50, 2560, 1024), (7, 16, 48)])
def test_gemm_bf16_matches_fp64(M, N, K):
    from yanlongvla_amd import kernels as Kn
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g, device=DEV).bfloat16()
    w = torch.randint(-127, 128, (N, K), generator=g, device=DEV).float().bfloat16()
    sw = torch.rand(N, generator=g, device=DEV) + 0.5
    ref = (a.double().cpu() @ w.double().cpu().t())
    z = Kn.gemm_bf16(a, w, torch.empty(M, N, device=DEV), sw=sw)
    zr = ref * sw.double().cpu()[None, :]
    assert ((z.double().cpu() - zr).norm() / zr.norm()).item() < 1e-6
    y = Kn.gemm_bf16(a, w, torch.empty(M, N, dtype=torch.bfloat16, device=DEV))
    z0 = Kn.gemm_bf16(a, w, torch.empty(M, N, device=DEV))
    assert np.array_equal(bits16(y), O.bf16_bits(z0.cpu().numpy()))              # BF16 output = RNE of the FP32 sums
    assert ((z0.double().cpu() - ref).norm() / ref.norm()).item() < 1e-6


@pytest.mark.parametrize('M,part', [(50, 'expert'), (1, 'expert'), (200, 'llm'), (16, 'llm')])
@pytest.mark.parametrize('mode', ['fly', 'resident'])
def test_group_float_path_matches_oracle(M, part, mode):
    """W2 float path of a q / k / v group against the oracle's restatement: relative L2 <= 2e-3 (FP32 device sums against
    FP64; the prefill variant rounds the product to BF16 before the row scale)."""
    from yanlongvla_amd.modules import Group, KLinear
    layers, oracles = qkv_layers(300 + M)
    g = Group(layers, part, mode, a8=False)
    mods = [KLinear(g, i) for i in range(3)]
    x = torch.randn(M, 1024, device=DEV).bfloat16()
    xs = x.float().cpu().numpy()
    for mod, ol in zip(mods, oracles):
        y = O.bf16_to_f32(bits16(mod(x)))
        ref = O.bf16_to_f32(O.w2_linear(xs, ol, part == 'expert'))
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 2e-3


def test_install_float_runtime():
    """install(a8=False): the W2 float path at the fly / resident / hybrid operating points gives the same chunk; MLPs and
    decoder layers stay unfused (the fused middles are W2A8 kernels)."""
    from yanlongvla_amd import gemma, modules
    outs, infos = {}, {}
    noise = torch.randn(50, 32, generator=torch.Generator(device=DEV).manual_seed(8), device=DEV)
    for runtime in ('fly', 'resident', 'hybrid'):
        model = small_expert()
        infos[runtime] = modules.install(model, runtime=runtime, a8=False, layers=gemma.synthetic_layers(model, 12, DEV))
        if runtime == 'hybrid':
            modules.decode_chunk(model)
        outs[runtime] = model.sample_chunk(noise, steps=2)
    assert infos['fly']['fused_mlps'] == 0 and infos['fly']['fused_layers'] == 0
    assert torch.equal(outs['fly'], outs['resident']) and torch.equal(outs['fly'], outs['hybrid'])
    assert torch.isfinite(outs['fly']).all()


# ------------------------------------------------------------------------------- row-group tables and GR00T shapes
@pytest.mark.parametrize('m,n,G', [(1536, 1536, 16), (3072, 1024, 16), (256, 512, 2), (6144, 1536, 8)])
def test_row_group_tables_bitexact(m, n, G):
    """(G, 512, 2) row-group tables: per-group snap, dense INT8 / FP16 decode, the fused small-M product (q / k / v-style
    Group at 50 tokens), the prefill path (200 tokens) and RefLinear, all bit-exact against the oracle."""
    from yanlongvla_amd import kernels as K
    from yanlongvla_amd.modules import Group, KLinear, RefLinear
    L, ol = device_layer(m, n, m + G, groups=G)
    assert L.groups == G
    assert np.array_equal(L.t8.cpu().numpy(), ol.t8) and np.array_equal(L.rs.cpu().numpy().view(np.uint32), ol.rs.view(np.uint32))
    assert np.array_equal(L.w8_reference().cpu().numpy(), ol.w8_reference())
    f16 = L.decode_f16()
    assert np.array_equal(f16.cpu().numpy(), O.lookup(ol.states(), ol.tlut.astype(np.float32)).astype(np.float16))
    for M, part in ((50, 'expert'), (200, 'llm')):
        x = torch.randn(M, n, device=DEV).bfloat16()
        ref = O.reference_linear(x.float().cpu().numpy(), ol)
        for mode in ('fly', 'resident'):
            y = KLinear(Group([L], part, mode), 0)(x)
            assert np.array_equal(bits16(y), ref), (M, mode)
        assert np.array_equal(bits16(RefLinear(L)(x)), ref)


@pytest.mark.parametrize('nl,M', [(1, 1), (3, 4), (300, 1)])
def test_row_group_tables_gemv(nl, M):
    """FP16-table decode-GEMV over layers with row-group tables (latency and layer-stream plans) against the oracle."""
    from yanlongvla_amd import kernels as K
    m, n, G = 512, 1024, 4
    layers = [device_layer(m, n, 900 + i, groups=G) for i in range(nl)]
    su = layers[0][0].su
    x = torch.randn(M, n, device=DEV).half()
    h16 = torch.empty(M, n, dtype=torch.float16, device=DEV)
    hs = torch.empty(M, dtype=torch.float32, device=DEV)
    K.pre_h16(x, su, h16, hs)
    zs = [torch.empty(M, m, device=DEV) for _ in layers]
    words = [L.words() for L, _ in layers]
    desc = K.gemv_descriptors([(w, L.tlut, L.row_scale, z) for w, (L, _), z in zip(words, layers, zs)])
    K.gemv_f16(desc, h16, hs, m, n, rows_per_table=m // G)
    xs = x.float().cpu().numpy()
    for (L, ol), z in list(zip(layers, zs))[:4] + list(zip(layers, zs))[-2:]:
        ol.su = su.cpu().numpy()
        y = torch.empty(M, m, device=DEV)
        K.post(z, None, None, L.sv, None, y)
        ref = O.reference_linear(xs, ol, a8=False, table='fp16', out_dtype='f32')
        assert np.linalg.norm(y.cpu().numpy() - ref) / np.linalg.norm(ref) < 2e-3
