"""Model integration: swaps the quantized nn.Linear modules of a policy for TCQ W2A8 modules running on the HIP library.

Mirrors deploy/tcq_kernels/modules.py (Group 29-155, KLinear 158-167, KGatedMLP 170-189, KPlainMLP 192-206, RefLinear
209-219, install 246-311, decode_chunk 314-320): same class and function names, arguments and operating points.

Runtimes (install(policy, row, runtime)):
  dense        BF16 dense weights in the original basis written into the existing nn.Linear modules
  reference    RefLinear: the layer definition as separate unfused steps (decode, rotate, quantize, exact GEMM, rotate)
  resident     operating point (i): every layer decoded once at load, weights held as INT8
  fly          operating point (ii): every layer decoded from the 2-bit stream on each call
  hybrid       operating point (iii): backbone on the fly; action expert decoded once per chunk (decode_chunk) into INT8

Layers that read the same tensor with identical input signs share one rotation + quantization and one product (q/k/v;
gate/up): the group runs on the first member's call and the other members return their slice.

Products by token count: up to SMALL_M tokens the small-M kernels (tcq_gemm_tcq on the stream / tcq_gemm_w8 on INT8
weights) give FP32 z = (acc * s) * rs directly; more tokens run the INT8 MFMA GEMM (tcq_gemm_i8) to exact int32 accumulators,
on the resident INT8 weights or on weights decoded for the call. Every launch goes to the HIP library; nothing here computes
with PyTorch ops except the bookkeeping (views, empty outputs).
"""
import torch

from . import kernels
from . import tcq_format as F

RUNTIMES = ('dense', 'reference', 'resident', 'fly', 'hybrid')
GROUPS = (('q_proj', 'k_proj', 'v_proj'), ('gate_proj', 'up_proj'))
STATS = dict(group_runs=0, regroup_misses=0, fused_mlps=0, fused_layers=0, chained_prologues=0)
# mlp: KGatedMLP / KPlainMLP; split: gated-MLP middle as postg + pre2 instead of one mid2 launch; layer: KDecoderLayer (norms
# and residual adds fused into the prologues / epilogues); chain: a decoder layer's last epilogue also computes the next
# layer's norm + rotate + quantize prologue
FUSE = dict(post3=True, mlp=True, split=False, layer=True, chain=True)
SMALL_M = 64                                         # most tokens of the small-M products


def part_of(name):
    return 'expert' if '.gemma_expert.' in name else 'vision' if 'vision_tower' in name else 'llm'


def is_quantizable(name, module):
    """The quantized Linear layers of the pi0.5 policy (baselines/common.py:51-58): encoder / language-model / expert layers;
    embeddings, projector, heads, action / time projections and norms stay dense."""
    if not isinstance(module, torch.nn.Linear):
        return False
    if name.endswith(('.input_layernorm.dense', '.post_attention_layernorm.dense')):
        return False
    return ('.vision_tower.vision_model.encoder.layers.' in name or '.language_model.layers.' in name or
            '.gemma_expert.model.layers.' in name)


class Group:
    """Layers sharing one input rotation + quantization and one product, columns side by side (modules.py:29-155).
    mode: resident (INT8 weights, stream released) | fly (decoded on every call) | chunk (INT8 weights re-decoded by
    decode_chunk); a8: INT8 activations, else the W2 float path (BF16 rotated activations, the INT8 table values as BF16
    weights, FP32 accumulation; modules.py:117-144)."""

    def __init__(self, layers, part, mode, a8=True):
        self.layers, self.part, self.mode, self.a8 = layers, part, mode, a8
        self.K = layers[0].n
        if not all(L.n == self.K and torch.equal(L.su, layers[0].su) for L in layers):
            raise ValueError(f'group members must share the input width and signs: {[L.name for L in layers]}')
        if len(layers) > kernels._lib.MAX_SEGS:
            raise ValueError(f'at most {kernels._lib.MAX_SEGS} layers per group')
        self.su = layers[0].su
        self.N = [L.m for L in layers]
        self.col0 = [sum(self.N[:i]) for i in range(len(layers))]
        self.Ntot = sum(self.N)
        self.small = part == 'expert'
        self.W = None
        self.rs = torch.cat([L.rs for L in layers]).contiguous()
        self.sv = torch.cat([L.sv for L in layers]).contiguous()
        self.bias = torch.cat([L.bias for L in layers]).contiguous() if layers[0].bias is not None else None
        self.rs_parts = [self.rs[c:c + n] for c, n in zip(self.col0, self.N)]
        self.sv_parts = [self.sv[c:c + n] for c, n in zip(self.col0, self.N)]
        self.bias_parts = [None if self.bias is None else self.bias[c:c + n] for c, n in zip(self.col0, self.N)]
        if not a8:                                          # BF16 bit patterns of the INT8 table values (modules.py:60)
            self.tb = [L.t8.to(torch.bfloat16).contiguous() for L in layers]
        if mode == 'chunk' and a8:
            for L in layers:
                if L.t8.dim() == 2:
                    L.words()                               # the per-chunk decode reads the repacked words
        if mode in ('resident', 'chunk'):
            self.W = torch.empty(self.Ntot, self.K, dtype=torch.int8 if a8 else torch.bfloat16, device=self.su.device)
            self.decode()
        elif a8:
            for L in layers:
                L.words()                                   # repack once at load: the fused small-M product reads it
        self.x = self.outs = None
        self.served = 0

    def decode(self, W=None):
        W = self.W if W is None else W
        for i, (L, c) in enumerate(zip(self.layers, self.col0)):
            if self.a8 and L.t8.dim() == 2 and L._words is not None:
                kernels.decode_words(L._words, L.t8, W[c:c + L.m])      # the repacked words the fused products keep
            elif self.a8:
                kernels.decode(L.bits, L.t8, W[c:c + L.m])
            else:
                kernels.decode_bf16(L.bits, self.tb[i], W[c:c + L.m])
        return W

    def prep(self, x):
        x2 = x.reshape(-1, self.K)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        if x2.dtype not in (torch.bfloat16, torch.float32, torch.float16):
            x2 = x2.float()
        return x2

    def buffers(self, M, dev):
        """Quantized activations and the per-token scales: up to SMALL_M tokens in the token-block layout the small-M products
        read fastest (q4), else (M, K) row-major (q)."""
        scale = torch.empty(M, dtype=torch.float32, device=dev)
        if M <= SMALL_M and self.K % 16 == 0:
            return dict(q=None, q4=kernels.token_blocks(M, self.K, dev), scale=scale)
        return dict(q=torch.empty(M, self.K, dtype=torch.int8, device=dev), q4=None, scale=scale)

    def quantize(self, x2):
        b = self.buffers(x2.shape[0], x2.device)
        kernels.pre(x2, self.su, q=b['q'], q4=b['q4'], scale=b['scale'])
        return b

    def product(self, b):
        """INT8 activations -> FP32 z = (float(acc) * s) * rs (M, Ntot) of the exact int32 product acc: few tokens on the
        fused decode products, many tokens on the INT8 MFMA GEMM with the scaling in its epilogue (the order of tcq_post)."""
        q = b['q'] if b['q'] is not None else b['q4']
        M, dev = b['scale'].numel(), q.device
        if M <= SMALL_M:
            z = torch.empty(M, self.Ntot, dtype=torch.float32, device=dev)
            if self.W is not None:
                segs = [(self.W[c:c + n], None, r, z[:, c:]) for c, n, r in zip(self.col0, self.N, self.rs_parts)]
                kernels.gemm_w8_segments(segs, q, b['scale'], self.Ntot)
            else:
                segs = [(L.words(), L.t8, r, z[:, c:]) for L, c, r in zip(self.layers, self.col0, self.rs_parts)]
                kernels.gemm_tcq_segments(segs, q, b['scale'], self.Ntot)
            return z
        W = self.W if self.W is not None else self.decode(torch.empty(self.Ntot, self.K, dtype=torch.int8, device=dev))
        z = torch.empty(M, self.Ntot, dtype=torch.float32, device=dev)
        return kernels.gemm_i8(q, W, z, sa=b['scale'], sw=self.rs)

    def posts(self, acc, b, shape, gelu0=False, outs=None):
        """acc: FP32 z (already scaled), INT32 (scaled here by the token scales of b and rs) or BF16 (scaled by rs).
        outs: per segment, None or a contiguous (M, n) BF16 tensor the segment's output is written to (e.g. a row of a
        preallocated key / value cache)."""
        M, dev = acc.shape[0], acc.device
        ys = [torch.empty(M, n, dtype=torch.bfloat16, device=dev) if outs is None or outs[i] is None else outs[i]
              for i, n in enumerate(self.N)]
        for y, n in zip(ys, self.N):
            if y.shape != (M, n) or y.dtype != torch.bfloat16 or not y.is_contiguous():
                raise ValueError(f'segment output {tuple(y.shape)} {y.dtype}: expected a contiguous ({M}, {n}) BF16 tensor')
        scaled = acc.dtype == torch.float32
        segs = [(acc, c, None if scaled else r, v, bb, y, gelu0 and i == 0)
                for i, (c, r, v, bb, y) in enumerate(zip(self.col0, self.rs_parts, self.sv_parts, self.bias_parts, ys))]
        kernels.post_group(segs, acc.dtype, torch.bfloat16, b['scale'] if acc.dtype == torch.int32 else None, M,
                           gelu_lut=kernels.gelu_table(dev) if gelu0 else None)
        return [y.reshape(*shape[:-1], n) for y, n in zip(ys, self.N)]

    def run(self, x):
        x2 = self.prep(x)
        if not self.a8:
            return self.run_float(x2, x.shape)
        b = self.quantize(x2)
        outs = self.posts(self.product(b), b, x.shape)
        STATS['group_runs'] += 1
        return outs

    def run_float(self, x2, shape):
        """W2: BF16 rotated activations (kernels.rht), BF16 weights decoded from the INT8 table values, FP32 accumulation
        (tcq_gemm_bf16). Expert: z = acc * rs in FP32; prefill: the product rounded to BF16, scaled by rs in the epilogue
        (modules.py:117-144)."""
        M, dev = x2.shape[0], x2.device
        h = torch.empty(M, self.K, dtype=torch.bfloat16, device=dev)
        kernels.rht(x2, self.su, h)
        W = self.W if self.W is not None else self.decode(torch.empty(self.Ntot, self.K, dtype=torch.bfloat16, device=dev))
        if self.small:
            acc = kernels.gemm_bf16(h, W, torch.empty(M, self.Ntot, dtype=torch.float32, device=dev), sw=self.rs)
        else:
            acc = kernels.gemm_bf16(h, W, torch.empty(M, self.Ntot, dtype=torch.bfloat16, device=dev))
        outs = self.posts(acc, None, shape)
        STATS['group_runs'] += 1
        return outs

    def get(self, x, index):
        if self.x is not x:
            if self.x is not None:
                STATS['regroup_misses'] += 1
            self.outs = self.run(x)
            self.x = x
            self.served = 0
        out = self.outs[index]
        self.served += 1
        if self.served == len(self.layers):
            self.x = self.outs = None
        return out


class KLinear(torch.nn.Module):
    """One member of a Group as an nn.Linear replacement (modules.py:158-167)."""

    def __init__(self, group, index):
        super().__init__()
        self.group, self.index = [group], index                 # list: keeps the group out of the module tree
        L = group.layers[index]
        self.in_features, self.out_features, self.layer_name = L.n, L.m, L.name
        self.register_buffer('weight', torch.empty(0, dtype=torch.bfloat16, device=L.su.device), persistent=False)

    def forward(self, x):
        return self.group[0].get(x, self.index)


class KGatedMLP(torch.nn.Module):
    """Gemma MLP down(gelu(gate(x)) * up(x)) with the middle fused (modules.py:170-189): rotate + quantize, product, middle
    (tcq_mid2, or postg + pre2 with FUSE['split']), product, scale + rotate."""

    def __init__(self, gate_up, down):
        super().__init__()
        self.groups = [gate_up, down]
        self.gate_proj, self.up_proj, self.down_proj = KLinear(gate_up, 0), KLinear(gate_up, 1), KLinear(down, 0)

    def forward(self, x):
        gu, down = self.groups
        b = gu.quantize(gu.prep(x))
        acc = gu.product(b)
        M, dev = acc.shape[0], acc.device
        b2 = down.buffers(M, dev)
        scaled = acc.dtype == torch.float32
        if FUSE['split']:
            g = torch.empty(M, gu.N[0], dtype=torch.bfloat16, device=dev)
            u = torch.empty_like(g)
            segs =[(acc, gu.col0[0], None if scaled else gu.rs_parts[0], gu.sv_parts[0], None, g, True),
                    (acc, gu.col0[1], None if scaled else gu.rs_parts[1], gu.sv_parts[1], None, u, False)]
            kernels.post_group(segs, acc.dtype, torch.bfloat16, None if scaled else b['scale'], M,
                               gelu_lut=kernels.gelu_table(dev))
            kernels.pre2(g, u, down.su, q=b2['q'], q4=b2['q4'], scale=b2['scale'])
        else:
            kernels.mid2(acc, None if scaled else b['scale'], None if scaled else gu.rs, gu.sv, down.su, q=b2['q'],
                         q4=b2['q4'], scale=b2['scale'])
        STATS['fused_mlps'] += 1
        return down.posts(down.product(b2), b2, x.shape)[0]


class KPlainMLP(torch.nn.Module):
    """SigLIP MLP fc2(gelu(fc1(x))) with the middle fused (modules.py:192-206)."""

    def __init__(self, fc1, fc2):
        super().__init__()
        self.groups = [fc1, fc2]
        self.fc1, self.fc2 = KLinear(fc1, 0), KLinear(fc2, 0)

    def forward(self, x):
        g1, g2 = self.groups
        b = g1.quantize(g1.prep(x))
        acc = g1.product(b)
        b2 = g2.buffers(acc.shape[0], acc.device)
        scaled = acc.dtype == torch.float32
        kernels.mid1(acc, None if scaled else b['scale'], None if scaled else g1.rs, g1.sv, g1.bias, g2.su, q=b2['q'],
                     q4=b2['q4'], scale=b2['scale'])
        STATS['fused_mlps'] += 1
        return g2.posts(g2.product(b2), b2, x.shape)[0]


class KDecoderLayer(torch.nn.Module):
    """Gemma decoder layer x + attn(norm1(x)) -> + mlp(norm2(.)) over the layer's groups with the norms and residual adds
    fused into the TCQ kernels: norm1 + rotate + quantize (tcq_norm_pre), q/k/v product, q/k/v epilogue, attention (the
    model's own), o rotate + quantize, o product, o epilogue + residual + norm2 + rotate + quantize (tcq_post_add_norm_pre),
    gate/up product, gated middle (tcq_mid2), down product, down epilogue + residual. Every rounding point is the unfused
    layer's, so the output equals the module-by-module forward bit for bit. No reference counterpart: it extends the
    reference's MLP fusion (modules.py:170-189) to the whole layer.

    Chained layers (install links the consecutive decoder layers of a stack): the down epilogue + residual also runs the
    next layer's norm1 + rotate + quantize on the residual output it writes, and leaves the result with the next layer.
    That layer takes it instead of launching tcq_norm_pre only when its input is that very output (same storage and shape;
    the hand-off keeps the output alive, so its memory cannot be reused meanwhile) and unmodified: same version counter,
    or, for inference tensors (torch.inference_mode keeps no version counters), the very object this layer returned. An
    in-place change of that returned object between two layers inside inference mode is the one case the check cannot
    see; FUSE['chain'] = False turns the hand-off off."""

    def __init__(self, layer, qkv, o, mlp):
        super().__init__()
        self.input_layernorm, self.post_attention_layernorm = layer.input_layernorm, layer.post_attention_layernorm
        self.self_attn, self.mlp = layer.self_attn, mlp
        self.groups = [qkv, o]
        self._next = []          # the following decoder layer of the stack (kept out of the module tree)
        self._handoff = None     # (residual output, its version, q / scale buffers) left by the previous layer

    def _prologue(self, x, x2):
        """The q/k/v input buffers the previous layer computed for exactly this input (x as passed, x2 its 2-D view), or
        None."""
        h, self._handoff = self._handoff, None
        if h is None:
            return None
        xo, ver, ret, b = h
        if x2.data_ptr() != xo.data_ptr() or x2.shape != xo.shape or x2.dtype != xo.dtype:
            return None
        if ver is None:
            return b if x is ret else None
        return b if (not x2.is_inference() and x2._version == ver) else None

    def forward(self, x, cache_k=None, cache_v=None, causal_offset=None, kv_out=None):
        """kv_out: None, or (k, v) contiguous (M, head_dim) BF16 tensors that this call's keys / values are written to by
        the q/k/v epilogue itself (the rows of a preallocated cache); they are then the returned k, v."""
        qkv, og = self.groups
        gu, dn = self.mlp.groups
        n1, n2 = self.input_layernorm, self.post_attention_layernorm
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        M, dev = x2.shape[0], x2.device
        b = self._prologue(x, x2)
        if b is None:
            b = qkv.buffers(M, dev)
            kernels.norm_pre(x2, n1.weight, n1.eps, qkv.su, q=b['q'], q4=b['q4'], scale=b['scale'])
        else:
            STATS['chained_prologues'] += 1
        q, k, v = qkv.posts(qkv.product(b), b, x2.shape, outs=None if kv_out is None else [None, kv_out[0], kv_out[1]])
        if hasattr(self.self_attn, 'core_quantized') and self.self_attn._device(q):
            b2 = og.buffers(M, dev)
            self.self_attn.core_quantized(q, k, v, cache_k, cache_v, causal_offset, og.su, b2['q'], b2['scale'], q4=b2['q4'])
        else:
            b2 = og.quantize(og.prep(self.self_attn.core(q, k, v, cache_k, cache_v, causal_offset)))
        z = og.product(b2)
        x3 = torch.empty_like(x2)
        b3 = gu.buffers(M, dev)
        sc = z.dtype == torch.float32
        kernels.post_add_norm_pre(z, None if sc else b2['scale'], None if sc else og.rs, og.sv, og.bias, x2, x3, n2.weight, n2.eps,
                                  gu.su, q=b3['q'], q4=b3['q4'], scale=b3['scale'])
        acc = gu.product(b3)
        b4 = dn.buffers(M, dev)
        sc = acc.dtype == torch.float32
        kernels.mid2(acc, None if sc else b3['scale'], None if sc else gu.rs, gu.sv, dn.su, q=b4['q'], q4=b4['q4'], scale=b4['scale'])
        z4 = dn.product(b4)
        x4 = torch.empty_like(x2)
        sc = z4.dtype == torch.float32
        nxt = self._next[0] if (self._next and FUSE['chain']) else None
        if nxt is None:
            kernels.post_add_norm_pre(z4, None if sc else b4['scale'], None if sc else dn.rs, dn.sv, dn.bias, x3, x4)
        else:
            nq, nn1 = nxt.groups[0], nxt.input_layernorm
            bn = nq.buffers(M, dev)
            kernels.post_add_norm_pre(z4, None if sc else b4['scale'], None if sc else dn.rs, dn.sv, dn.bias, x3, x4,
                                      nn1.weight, nn1.eps, nq.su, q=bn['q'], q4=bn['q4'], scale=bn['scale'])
        out = x4.reshape(shape)
        if nxt is not None:
            nxt._handoff = (x4, None if x4.is_inference() else x4._version, out, bn)
        STATS['fused_layers'] += 1
        return out, k, v


class RefLinear(torch.nn.Module):
    """The layer by definition, one unfused step per launch (modules.py:209-219 runs tcq_format.reference_linear):
    a8 / INT8 table: h = fwht(x * su) in FP32 -> per-token INT8 -> exact int32 product with the decoded INT8 weight ->
    (acc * s) * rs -> fwht -> * sv (+ bias) -> BF16. a8=False: the FP32 rotated activations times the decoded weight of
    `table` in FP64, * row scale, then the same output rotation. resident=False decodes on every call."""

    def __init__(self, layer, a8=True, table='int8', resident=True):
        super().__init__()
        if table not in ('int8', 'fp16') or (a8 and table != 'int8'):
            raise ValueError('RefLinear: a8 needs the INT8 table; table is int8 or fp16')
        self.layer, self.a8, self.table, self.resident = [layer], a8, table, resident
        self.w8 = layer.w8_reference() if (table == 'int8' and resident) else None
        self.in_features, self.out_features, self.layer_name = layer.n, layer.m, layer.name
        self.register_buffer('weight', torch.empty(0, dtype=torch.bfloat16, device=layer.su.device), persistent=False)

    def forward(self, x):
        L = self.layer[0]
        shape = x.shape
        x2 = x.reshape(-1, L.n).contiguous()
        if x2.dtype not in (torch.bfloat16, torch.float32, torch.float16):
            x2 = x2.float()
        M, dev = x2.shape[0], x2.device
        h = torch.empty(M, L.n, dtype=torch.float32, device=dev)
        kernels.rht(x2, L.su, h)
        if self.a8:
            q = torch.empty(M, L.n, dtype=torch.int8, device=dev)
            s = torch.empty(M, dtype=torch.float32, device=dev)
            kernels.quantize_rows(h, q, s)
            w8 = self.w8 if self.w8 is not None else L.w8_reference()
            acc = kernels.gemm_i8(q, w8, torch.empty(M, L.m, dtype=torch.int32, device=dev))
            y = torch.empty(M, L.m, dtype=torch.bfloat16, device=dev)
            kernels.post(acc, s, L.rs, L.sv, L.bias, y)
        else:
            w = (self.w8 if self.w8 is not None else L.w8_reference()) if self.table == 'int8' else L.decode_f16()
            r = L.rs if self.table == 'int8' else L.row_scale.float()
            z = ((h.double() @ w.double().t()).float() * r[None, :]).contiguous()
            y = torch.empty(M, L.m, dtype=torch.bfloat16, device=dev)
            kernels.post(z, None, None, L.sv, L.bias, y)
        return y.reshape(*shape[:-1], L.m)


def set_submodule(model, name, module):
    parent, _, leaf = name.rpartition('.')
    setattr(model.get_submodule(parent) if parent else model, leaf, module)


def apply_row_state(model, row):
    """The fine-tuned norm weights stored beside the packed file (dense.safetensors entries norm::<module>::<attr>,
    modules.py:231-243). The reference's row-INT8 token embedding belongs to its private policy loader and is not applied."""
    path = F.packed_path(row).with_name('dense.safetensors')
    if not path.exists():
        return 0
    from safetensors import safe_open
    norms = 0
    with safe_open(str(path), framework='pt', device='cpu') as f:
        for k in sorted(f.keys()):
            if k.startswith('norm::'):
                _, name, attr = k.split('::')
                p = getattr(model.get_submodule(name), attr)
                v = f.get_tensor(k)
                if v.shape != p.shape or v.dtype != p.dtype:
                    raise ValueError(f'{k}: {tuple(v.shape)} {v.dtype} does not match {tuple(p.shape)} {p.dtype}')
                p.data.copy_(v)
                norms += 1
    return norms


def install(policy, row=F.ROW, runtime='resident', a8=True, table='int8', reference_resident=True, layers=None):
    """Swap every quantizable nn.Linear of policy (or policy._model) found in the packed file of `row` (modules.py:246-311).
    layers: an already loaded {name: Layer} to use instead of reading the file."""
    if runtime not in RUNTIMES:
        raise ValueError(f'runtime {runtime!r} not in {RUNTIMES}')
    model = getattr(policy, '_model', policy)
    if layers is None:
        stored = set(F.layer_names(row))
        names = [n for n, m in model.named_modules() if n in stored and is_quantizable(n, m)]
    else:
        names = list(layers)
    norms = apply_row_state(model, row) if layers is None else 0
    info = dict(row=str(row), runtime=runtime, layers=len(names), norm_tensors=norms)
    biases = {}
    for name in names:
        m = model.get_submodule(name)
        if not isinstance(m, torch.nn.Linear):
            raise TypeError(f'{name}: {type(m).__name__} is not an nn.Linear')
        if m.bias is not None:
            biases[name] = m.bias.detach().float().clone()
    if layers is None:
        dev = next(model.parameters()).device
        layers = F.load(row, device=dev, names=names, biases=biases)
    else:
        for n, b in biases.items():
            if layers[n].bias is None:
                layers[n].bias = b.to(layers[n].su.device).contiguous()
    if runtime == 'dense':
        for name in names:
            m = model.get_submodule(name)
            w = layers[name].dense(table)
            if m.weight.shape != w.shape:
                raise ValueError(f'{name}: weight {tuple(m.weight.shape)} != {tuple(w.shape)}')
            m.weight.data.copy_(w.to(m.weight.dtype))
        return info
    if runtime == 'reference':
        for name in names:
            set_submodule(model, name, RefLinear(layers[name], a8=a8, table=table, resident=reference_resident))
        return info
    groups, done = [], set()
    for name in names:
        if name in done:
            continue
        parent, _, leaf = name.rpartition('.')
        members = [name]
        for g in GROUPS:
            if leaf in g:
                cand = [f'{parent}.{x}' for x in g]
                if all(c in layers for c in cand) and all(layers[c].n == layers[cand[0]].n and
                                                          torch.equal(layers[c].su, layers[cand[0]].su) for c in cand):
                    members = cand
        part = part_of(name)
        mode = 'resident' if runtime == 'resident' else 'fly' if (runtime == 'fly' or part != 'expert') else 'chunk'
        group = Group([layers[n] for n in members], part, mode, a8=a8)
        for i, n in enumerate(members):
            set_submodule(model, n, KLinear(group, i))
            done.add(n)
        if mode == 'resident':
            for L in group.layers:
                L.bits_resident = False
                L.bits = None                                   # resident: the bitstream is not needed after load
                L._words = None
        groups.append(group)
    fused = 0
    if a8 and FUSE['mlp']:
        by_name = {g.layers[0].name: g for g in groups}
        for g in list(groups):
            parent, _, leaf = g.layers[0].name.rpartition('.')
            if leaf == 'gate_proj' and len(g.layers) == 2 and f'{parent}.down_proj' in by_name:
                if type(model.get_submodule(parent)).__name__ != 'GemmaMLP':
                    raise TypeError(f'{parent}: expected a GemmaMLP, got {type(model.get_submodule(parent)).__name__}')
                set_submodule(model, parent, KGatedMLP(g, by_name[f'{parent}.down_proj']))
                fused += 1
            elif leaf == 'fc1' and f'{parent}.fc2' in by_name:
                if type(model.get_submodule(parent)).__name__ != 'SiglipMLP':
                    raise TypeError(f'{parent}: expected a SiglipMLP, got {type(model.get_submodule(parent)).__name__}')
                set_submodule(model, parent, KPlainMLP(g, by_name[f'{parent}.fc2']))
                fused += 1
    layers_fused = 0
    if a8 and FUSE['mlp'] and FUSE['layer']:
        by_name = {g.layers[0].name: g for g in groups}
        for g in groups:
            attn, _, leaf = g.layers[0].name.rpartition('.')
            lname = attn.rpartition('.')[0]
            if leaf != 'q_proj' or len(g.layers) != 3 or f'{attn}.o_proj' not in by_name:
                continue
            layer = model.get_submodule(lname)
            mlp = getattr(layer, 'mlp', None)
            if type(layer).__name__ != 'GemmaDecoderLayer' or not isinstance(mlp, KGatedMLP) or not hasattr(layer.self_attn, 'core'):
                continue
            set_submodule(model, lname, KDecoderLayer(layer, g, by_name[f'{attn}.o_proj'], mlp))
            layers_fused += 1
        for ml in model.modules():                     # link consecutive decoder layers of each stack
            if isinstance(ml, torch.nn.ModuleList):
                for a, b in zip(ml[:-1], ml[1:]):
                    if isinstance(a, KDecoderLayer) and isinstance(b, KDecoderLayer):
                        a._next = [b]
    torch.cuda.synchronize()
    policy._tcq_groups = groups
    info['fused_layers'] = layers_fused
    info['fused_mlps'] = fused
    info.update(groups=len(groups), shared_rotations=sum(len(g.layers) - 1 for g in groups),
                modes={m: sum(1 for g in groups if g.mode == m) for m in ('resident', 'fly', 'chunk')})
    return info


def decode_chunk(policy):
    """Operating point (iii): decode the action expert's layers once per action chunk, before the first denoising step
    (modules.py:314-320). Returns the number of layers decoded."""
    n = 0
    for g in getattr(policy, '_tcq_groups', ()):
        if g.mode == 'chunk':
            g.decode()
            n += len(g.layers)
    return n
