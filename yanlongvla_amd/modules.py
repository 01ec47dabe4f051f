"""Model integration: puts the TCQ W2A8 deploy path behind a policy's quantized nn.Linear modules.

Drop-in counterpart of deploy/tcq_kernels/modules.py: the same public names and arguments (install 246-311, Group 29-155,
KLinear 158-167, KGatedMLP 170-189, KPlainMLP 192-206, RefLinear 209-219, decode_chunk 314-320), the same runtimes and
operating points, the same STATS counters. The bodies are this package's own: layers are planned into groups by bucket,
a group keeps one segment record per member, and the first-member-computes protocol is a pending-result record.

Runtimes (install(policy, row, runtime)):
  dense        BF16 dense weights in the original basis, written into the existing nn.Linear modules
  reference    RefLinear: the layer definition as separate unfused launches (decode, rotate, quantize, exact GEMM, rotate)
  resident     operating point (i): every layer decoded once at load, weights held as INT8
  fly          operating point (ii): every layer decoded from the 2-bit stream on each call
  hybrid       operating point (iii): backbone on the fly; action expert decoded once per chunk (decode_chunk) into INT8

Policies: the pi0.5 layer rule (baselines/common.py:51-58) and the GR00T N1.7 rule (baselines/groot/groot_common.py:33-42,
70-79; 432 Linear) are both known; install picks the one whose layer names the model carries. GR00T records may be
one-sided (no output rotation) and may carry column scales (groot_tcq.py:178-191).

Layers that read the same tensor with the same input signs share one rotation + quantization and one product (q/k/v,
gate/up): the group computes on the first member's call and the other members take their slice. Every launch goes to the
HIP library; nothing here computes with PyTorch ops except the bookkeeping (views, empty outputs).
"""
import contextlib
from collections import Counter, namedtuple
from itertools import accumulate

import torch

from . import kernels
from . import tcq_format as F

RUNTIMES = ('dense', 'reference', 'resident', 'fly', 'hybrid')
GROUPS = (('q_proj', 'k_proj', 'v_proj'), ('gate_proj', 'up_proj'))
STATS = dict(group_runs=0, regroup_misses=0, fused_mlps=0, fused_layers=0, chained_prologues=0, spread_middles=0,
             layer_prologues=0, pre_prologues=0, deferred_outputs=0, attn_prologues=0, attn_posts=0)
# mlp: KGatedMLP / KPlainMLP; split: gated-MLP middle as postg + pre2 instead of one mid2 launch; layer: KDecoderLayer (norms
# and residual adds fused into the prologues / epilogues); chain: a decoder layer's last epilogue also computes the next
# layer's norm + rotate + quantize prologue; spread: the 16384-wide gated-MLP middle of few tokens spread over many CUs
# (the first Walsh stages in the gate/up product, the rest in glu_split, then the down projection's pre) instead of mid2;
# prologue: at one token the o epilogue + residual + norm2 + rotate + quantize run inside the gate/up product's launch;
# pre_prologue: after the spread middle the down projection's rotate + quantize runs inside its product's launch;
# defer: inside deferred_outputs(), a layer's down epilogue + the next layer's norm1 prologue run in the next q/k/v product
# attn_prologue: at one token the attention's chunk merge + o rotate + quantize run inside the o product's launch;
# attn_post: with it, the q/k/v epilogue (output rotations, the new key / value rows) runs inside the attention's launch
FUSE = dict(post3=True, mlp=True, split=False, layer=True, chain=True, k_parts=True, spread=True, prologue=True,
            pre_prologue=True, defer=True, attn_prologue=True, attn_post=True)
SMALL_M = 64                                         # most tokens of the small-M products


# ------------------------------------------------------------------------------------------------------ layer rules
def part_of(name):
    """pi0.5 policy part of a layer name: the action expert, the vision tower or the language model."""
    if '.gemma_expert.' in name:
        return 'expert'
    return 'vision' if 'vision_tower' in name else 'llm'


_PI05_STACKS = ('.vision_tower.vision_model.encoder.layers.', '.language_model.layers.', '.gemma_expert.model.layers.')
_PI05_DENSE_TAILS = ('.input_layernorm.dense', '.post_attention_layernorm.dense')


def is_quantizable(name, module):
    """The quantized Linear layers of the pi0.5 policy (baselines/common.py:51-58): encoder / language-model / expert
    layers; embeddings, projector, heads, action / time projections and the norms' dense layers stay dense."""
    return (isinstance(module, torch.nn.Linear) and any(s in name for s in _PI05_STACKS)
            and not name.endswith(_PI05_DENSE_TAILS))


_GROOT_PARTS = (('backbone', ('backbone.model.model.visual.', 'backbone.model.model.language_model.layers.')),
                ('head', ('action_head.vl_self_attention.', 'action_head.model.transformer_blocks.')))
_GROOT_DENSE = ('norm1.linear', 'proj_out', 'lm_head', 'embed')


def groot_part_of(name):
    """GR00T N1.7 part of a layer name (groot_common.py:33-34, 57-62): 'backbone', 'head' or None."""
    return next((part for part, prefixes in _GROOT_PARTS if name.startswith(prefixes)), None)


def groot_is_quantizable(name, module):
    """The 432 quantized Linear layers of GR00T N1.7 (groot_common.py:35-42, 65-66): vision tower and LLM layers 0-15 of
    the backbone, vl_self_attention and the DiT blocks of the action head; the timestep-only AdaLN linears, proj_out_*,
    lm_head and embeddings stay dense."""
    return (isinstance(module, torch.nn.Linear) and groot_part_of(name) is not None
            and not any(d in name for d in _GROOT_DENSE))


Rule = namedtuple('Rule', 'name quantizable part streamed families')
# streamed(part): under the hybrid runtime the action-generating part is decoded per action chunk ('chunk'), the rest
# streams ('fly'). families: leaf names whose layers may share one input rotation.
PI05 = Rule('pi0.5', is_quantizable, part_of, lambda p: p != 'expert', GROUPS)
GROOT = Rule('gr00t', groot_is_quantizable, lambda n: groot_part_of(n) or 'backbone', lambda p: p != 'head',
             GROUPS + (('to_q', 'to_k', 'to_v'),))


def rule_for(model):
    """GR00T's rule for a model carrying GR00T layer names, else pi0.5's."""
    groot = any(groot_part_of(n) for n, _ in model.named_modules())
    return GROOT if groot else PI05


# ---------------------------------------------------------------------------------------------------------- groups
Segment = namedtuple('Segment', 'col0 width rs sv bias')     # one member's columns and epilogue vectors


def _shares_input(layers):
    """Members of a group read one rotated, quantized input: same width, input signs and column scales."""
    a = layers[0]

    def same(t, u):
        return (t is None and u is None) or (t is not None and u is not None and torch.equal(t, u))
    return all(L.n == a.n and torch.equal(L.su, a.su) and same(L.col_scale, a.col_scale) for L in layers)


def _cat(tensors):
    return None if tensors[0] is None else torch.cat(list(tensors)).contiguous()


class _Pending:
    """Outputs of one group run waiting for the members that have not taken theirs yet."""
    __slots__ = ('x', 'outs', 'waiting')

    def __init__(self, x, outs, taken):
        self.x, self.outs = x, outs
        self.waiting = set(range(len(outs))) - {taken}


class Group:
    """Layers sharing one input rotation + quantization and one product, their output columns side by side
    (modules.py:29-155). mode: resident (INT8 weights, stream released) | fly (decoded on every call) | chunk (INT8 weights
    re-decoded by decode_chunk); a8: INT8 activations, else the W2 float path (BF16 rotated activations, the INT8 table
    values as BF16 weights, FP32 accumulation; modules.py:117-144). Both paths keep the same weights: the packed words
    (fly), or INT8 weights (resident, chunk)."""

    def __init__(self, layers, part, mode, a8=True):
        if not _shares_input(layers):
            raise ValueError(f'group members must share the input width, signs and column scales: {[L.name for L in layers]}')
        if len(layers) > kernels._lib.MAX_SEGS:
            raise ValueError(f'at most {kernels._lib.MAX_SEGS} layers per group')
        sided = {L.sv is None for L in layers}
        if len(sided) > 1:
            raise ValueError(f'group mixes one-sided and two-sided layers: {[L.name for L in layers]}')
        self.layers, self.part, self.mode, self.a8 = list(layers), part, mode, a8
        lead = layers[0]
        self.K, self.su, self.col_scale = lead.n, lead.su, lead.col_scale
        if self.col_scale is not None and not a8:
            raise NotImplementedError('the W2 float path takes no column scales')
        self.one_sided = lead.sv is None
        self.N = [L.m for L in layers]
        self.col0 = list(accumulate([0] + self.N[:-1]))
        self.Ntot = sum(self.N)
        self.small = part in ('expert', 'head')           # the few-token (action-generating) part
        self.rs = _cat([L.rs for L in layers])
        self.sv = None if self.one_sided else _cat([L.sv for L in layers])
        self.bias = _cat([L.bias for L in layers]) if lead.bias is not None else None

        def piece(t, c, n):
            return None if t is None else t[c:c + n]
        self.segments = [Segment(c, n, piece(self.rs, c, n), piece(self.sv, c, n), piece(self.bias, c, n))
                         for c, n in zip(self.col0, self.N)]
        self.W = None
        if mode in ('resident', 'chunk'):
            if mode == 'chunk':
                self._repack()                              # the per-chunk decode reads the repacked words
            self.W = torch.empty(self.Ntot, self.K, dtype=torch.int8, device=self.su.device)
            self.decode()
        else:
            self._repack()                                  # the fused products read the repacked words
        self.pending = None

    def _repack(self):
        for L in self.layers:
            if L.t8.dim() == 2 or self.mode != 'chunk':
                L.words()

    # -------------------------------------------------------------------------------------------------- weights
    def decode(self, W=None):
        """The group's dense INT8 weight rows into W (default: the resident W)."""
        W = self.W if W is None else W
        for L, seg in zip(self.layers, self.segments):
            rows = W[seg.col0:seg.col0 + seg.width]
            if L.t8.dim() == 2 and L._words is not None:
                kernels.decode_words(L._words, L.t8, rows)          # the words the fused products keep
            else:
                kernels.decode(L.bits, L.t8, rows)
        return W

    # -------------------------------------------------------------------------------------------- activations
    def prep(self, x):
        """The (M, K) contiguous view of x in a dtype the rotation kernels read."""
        x2 = x.reshape(-1, self.K)
        if x2.dtype not in (torch.bfloat16, torch.float32, torch.float16):
            x2 = x2.float()
        return x2 if x2.is_contiguous() else x2.contiguous()

    def buffers(self, M, dev):
        """Quantized activations and per-token scales: up to SMALL_M tokens in the token-block layout the small-M products
        read fastest (q4), else (M, K) row-major (q)."""
        blocks = M <= SMALL_M and self.K % 16 == 0
        return dict(q=None if blocks else torch.empty(M, self.K, dtype=torch.int8, device=dev),
                    q4=kernels.token_blocks(M, self.K, dev) if blocks else None,
                    scale=torch.empty(M, dtype=torch.float32, device=dev))

    def quantize(self, x2):
        b = self.buffers(x2.shape[0], x2.device)
        kernels.pre(x2, self.su, q=b['q'], q4=b['q4'], scale=b['scale'], col_scale=self.col_scale)
        return b

    # ------------------------------------------------------------------------------------------------ product
    def k_parts(self, M):
        """K parts for a product of M tokens whose epilogue takes them (post_add_norm_pre): parts double while the
        product's workgroups (one per tile row and part) stay below the 256 CUs and every part keeps at least 4 of the
        256-column chunks; 1 for many tokens or when FUSE['k_parts'] is off. Measured on MI355X, product + epilogue:
        2048 x 16384 at one token 13.6 -> 12.4 us (fly), 19.3 -> 14.3 (resident INT8); 1024 x 4096 at 50 tokens (4 parts)
        12.4 -> 10.6 / 12.5 -> 9.7; 2048 x 2048 at one token unchanged. The epilogue adds K parts only for power-of-two
        rows of 1024 .. 16384 (its register engines), so every other output width keeps one part."""
        w = self.Ntot
        if not FUSE['k_parts'] or M > SMALL_M or w & (w - 1) or not 1024 <= w <= 16384:
            return 1
        tiles, nch = self.Ntot // 16, (self.K + 255) // 256
        parts = 1
        while parts < 4 and tiles * parts < 256 and nch >= 8 * parts:
            parts *= 2
        return parts

    def product(self, b, parts=1, pro=None):
        """INT8 activations -> FP32 z = (float(acc) * s) * rs (M, Ntot) of the exact int32 product acc: few tokens on the
        fused decode products, many tokens on the INT8 MFMA GEMM with the scaling in its epilogue (the order of tcq_post).
        parts 2 / 4 (few tokens): the int32 K parts of acc instead, (parts, M, Ntot), for post_add_norm_pre. pro: one token
        whose activations the decoder-layer prologue computes inside the product's launch (kernels.prologue; b unused)."""
        if pro is not None:                       # FP32 z after the layer prologue, int32 sums after the rotate + quantize one
            dev = self.rs.device
            layer = pro[0].acc is not None
            z = torch.empty(1, self.Ntot, dtype=torch.float32, device=dev) if layer else \
                torch.empty(parts, 1, self.Ntot, dtype=torch.int32, device=dev)
            out = z if layer else z[0]
            if self.W is not None:
                segs = [(self.W[s.col0:s.col0 + s.width], None, s.rs, out[:, s.col0:]) for s in self.segments]
            else:
                segs = [(L.words(), L.t8, s.rs, out[:, s.col0:]) for L, s in zip(self.layers, self.segments)]
            kernels.SmallProduct(segs, self.Ntot, resident=self.W is not None).run_pro(pro, parts)
            return z if (layer or parts > 1) else z[0]
        q = b['q'] if b['q'] is not None else b['q4']
        M, dev = b['scale'].numel(), q.device
        if parts > 1:
            if M > SMALL_M:
                raise ValueError(f'K parts are for at most {SMALL_M} tokens')
            acc = torch.empty(parts, M, self.Ntot, dtype=torch.int32, device=dev)
            if self.W is not None:
                segs = [(self.W[s.col0:s.col0 + s.width], None, s.rs, acc[0, :, s.col0:]) for s in self.segments]
                kernels.gemm_w8_segments(segs, q, b['scale'], self.Ntot, parts)
            else:
                segs = [(L.words(), L.t8, s.rs, acc[0, :, s.col0:]) for L, s in zip(self.layers, self.segments)]
                kernels.gemm_tcq_segments(segs, q, b['scale'], self.Ntot, parts)
            return acc
        z = torch.empty(M, self.Ntot, dtype=torch.float32, device=dev)
        if M > SMALL_M:
            W = self.W if self.W is not None else self.decode(torch.empty(self.Ntot, self.K, dtype=torch.int8, device=dev))
            return kernels.gemm_i8(q, W, z, sa=b['scale'], sw=self.rs)
        if self.W is not None:
            segs = [(self.W[s.col0:s.col0 + s.width], None, s.rs, z[:, s.col0:]) for s in self.segments]
            kernels.gemm_w8_segments(segs, q, b['scale'], self.Ntot)
        else:
            segs = [(L.words(), L.t8, s.rs, z[:, s.col0:]) for L, s in zip(self.layers, self.segments)]
            kernels.gemm_tcq_segments(segs, q, b['scale'], self.Ntot)
        return z

    def spreads(self, M):
        """Whether this gate | up group's middle at M tokens runs spread over many CUs (gemm_tcq_w128t + glu_split + pre):
        the fused decode of two 16384-wide members with one table each, K <= 4096, at most 16 tokens."""
        return (FUSE['spread'] and self.W is None and M <= 16 and self.K <= 4096 and self.N == [16384, 16384]
                and not self.one_sided and self.col_scale is None and all(L.t8.dim() == 2 for L in self.layers))

    def gated_middle(self, b, down, b2, pro=None):
        """This gate | up group's product and the GeGLU middle (tcq_mid2's operations) into the down projection's quantized
        input buffers b2: spread over many CUs when self.spreads(M), else one product launch and one mid2 launch. pro: one
        token whose input the decoder-layer prologue computes inside the product (kernels.prologue; b None)."""
        M, dev = (1, self.rs.device) if pro is not None else (b['scale'].numel(), b['scale'].device)
        if self.spreads(M):
            zt = torch.empty(2, M, 128, 128, dtype=torch.float32, device=dev)
            segs = [(L.words(), L.t8, s.rs, zt[i]) for i, (L, s) in enumerate(zip(self.layers, self.segments))]
            if pro is not None:
                kernels.gemm_tcq_w128t(segs, None, None, pro=pro)
            else:
                kernels.gemm_tcq_w128t(segs, b['q'] if b['q'] is not None else b['q4'], b['scale'])
            p = kernels.glu_split(zt, self.sv, kernels.gelu_table(dev), torch.empty(M, 16384, dtype=torch.bfloat16, device=dev))
            kernels.pre(p, down.su, q=b2['q'], q4=b2['q4'], scale=b2['scale'])
            STATS['spread_middles'] += 1
            return
        acc = self.product(b, pro=pro)
        s_tok, rs = (None, None) if acc.dtype == torch.float32 else (b['scale'], self.rs)
        kernels.mid2(acc, s_tok, rs, self.sv, down.su, q=b2['q'], q4=b2['q4'], scale=b2['scale'])

    def pre_prologue_fits(self, M):
        """Whether this group's product at M tokens can take a rotate + quantize prologue (tcq_gemm_*_pro without acc): one
        token, 16384 input columns, plain signs (no column scale)."""
        return FUSE['pre_prologue'] and M == 1 and self.a8 and self.K == 16384 and self.col_scale is None

    def gated_down(self, b, down, parts=1, pro=None):
        """This gate | up group's product, the GeGLU middle and the down projection's product: (z, b2) with z as
        down.product(b2, parts) returns it and b2 the down input's buffers (its token scale for the epilogue). On the
        spread middle at one token the down projection's rotate + quantize runs inside its product's launch (every
        workgroup computes the INT8 row from glu_split's output); else gated_middle then down.product. pro: as in
        gated_middle."""
        M, dev = (1, self.rs.device) if pro is not None else (b['scale'].numel(), b['scale'].device)
        if self.spreads(M) and down.pre_prologue_fits(M):
            zt = torch.empty(2, M, 128, 128, dtype=torch.float32, device=dev)
            segs = [(L.words(), L.t8, s.rs, zt[i]) for i, (L, s) in enumerate(zip(self.layers, self.segments))]
            if pro is not None:
                kernels.gemm_tcq_w128t(segs, None, None, pro=pro)
            else:
                kernels.gemm_tcq_w128t(segs, b['q'] if b['q'] is not None else b['q4'], b['scale'])
            p = kernels.glu_split(zt, self.sv, kernels.gelu_table(dev), torch.empty(M, 16384, dtype=torch.bfloat16, device=dev))
            b2 = dict(q=None, q4=None, scale=torch.empty(M, dtype=torch.float32, device=dev))
            z = down.product(None, parts, pro=kernels.prologue_pre(p, down.su, scale=b2['scale']))
            STATS['spread_middles'] += 1
            STATS['pre_prologues'] += 1
            return z, b2
        b2 = down.buffers(M, dev)
        self.gated_middle(b, down, b2, pro=pro)
        return down.product(b2, parts), b2

    # ------------------------------------------------------------------------------------------------ epilogue
    def posts(self, acc, b, shape, gelu0=False, outs=None):
        """acc: FP32 z (already scaled), INT32 (scaled here by the token scales of b and rs) or BF16 (scaled by rs).
        outs: per segment, None or a contiguous (M, n) BF16 tensor the segment's output is written to (e.g. a row of a
        preallocated key / value cache)."""
        M, dev = acc.shape[0], acc.device
        ys = []
        for i, s in enumerate(self.segments):
            y = outs[i] if outs is not None and outs[i] is not None else torch.empty(M, s.width, dtype=torch.bfloat16, device=dev)
            if y.shape != (M, s.width) or y.dtype != torch.bfloat16 or not y.is_contiguous():
                raise ValueError(f'segment output {tuple(y.shape)} {y.dtype}: expected a contiguous ({M}, {s.width}) BF16 tensor')
            ys.append(y)
        scaled = acc.dtype == torch.float32
        s_tok = b['scale'] if acc.dtype == torch.int32 else None
        if self.one_sided:                        # no output rotation: one plain epilogue per member
            if gelu0:
                raise ValueError('one-sided groups have no fused GELU epilogue')
            for s, y in zip(self.segments, ys):
                kernels.post(acc, s_tok, None if scaled else s.rs, None, s.bias, y, col0=s.col0)
        else:
            segs = [(acc, s.col0, None if scaled else s.rs, s.sv, s.bias, y, gelu0 and i == 0)
                    for i, (s, y) in enumerate(zip(self.segments, ys))]
            kernels.post_group(segs, acc.dtype, torch.bfloat16, s_tok, M,
                               gelu_lut=kernels.gelu_table(dev) if gelu0 else None)
        return [y.reshape(*shape[:-1], s.width) for s, y in zip(self.segments, ys)]

    # --------------------------------------------------------------------------------------------------- runs
    def run(self, x):
        """All members' outputs for input x."""
        x2 = self.prep(x)
        if self.a8:
            b = self.quantize(x2)
            outs = self.posts(self.product(b), b, x.shape)
        else:
            outs = self.run_float(x2, x.shape)
        STATS['group_runs'] += 1
        return outs

    def run_float(self, x2, shape):
        """W2: BF16 rotated activations (kernels.rht = the reference's pre_h), the INT8 table values as BF16 weights, FP32
        sums, on the fused products (kernels.gemmf_segments: the packed words decoded on the fly, or the resident INT8
        weights; no dense BF16 copy). Expert: z = acc * rs in FP32; prefill: the product rounded to BF16, scaled by rs in
        the epilogue (modules.py:117-144)."""
        M, dev = x2.shape[0], x2.device
        h = kernels.rht(x2, self.su, torch.empty(M, self.K, dtype=torch.bfloat16, device=dev))
        acc = torch.empty(M, self.Ntot, dtype=torch.float32 if self.small else torch.bfloat16, device=dev)
        if self.W is not None:
            segs = [(self.W[s.col0:s.col0 + s.width], None, s.rs, acc[:, s.col0:]) for s in self.segments]
        else:
            segs = [(L.words(), L.t8, s.rs, acc[:, s.col0:]) for L, s in zip(self.layers, self.segments)]
        kernels.gemmf_segments(segs, h, self.Ntot, resident=self.W is not None)
        return self.posts(acc, None, shape)

    def get(self, x, index):
        """Member index's output for input x. The first member called with a new input runs the group; the others take
        their slice of that run. A member asking again, or asking with another input, starts a new run (regroup_misses
        counts runs that replaced unfinished ones)."""
        p = self.pending
        if p is None or p.x is not x or index not in p.waiting:
            if p is not None:
                STATS['regroup_misses'] += 1
            p = self.pending = _Pending(x, self.run(x), index)
        else:
            p.waiting.discard(index)
        out = p.outs[index]
        if not p.waiting:
            self.pending = None
        return out


class KLinear(torch.nn.Module):
    """One member of a Group as an nn.Linear replacement (modules.py:158-167): in_features / out_features / layer_name of
    its layer, and an empty BF16 weight buffer the model reads only for its dtype."""

    def __init__(self, group, index):
        super().__init__()
        layer = group.layers[index]
        self.group = [group]                     # a list keeps the group out of the module tree
        self.index = index
        self.in_features, self.out_features, self.layer_name = layer.n, layer.m, layer.name
        self.register_buffer('weight', torch.empty(0, dtype=torch.bfloat16, device=layer.su.device), persistent=False)

    def forward(self, x):
        (group,) = self.group
        return group.get(x, self.index)


# ---------------------------------------------------------------------------------------------------- fused MLPs
def _first_half(group, x):
    """Rotate + quantize the MLP input and run the first product: (FP32 z, the quantized-input buffers)."""
    b = group.quantize(group.prep(x))
    return group.product(b), b


class KGatedMLP(torch.nn.Module):
    """Gemma MLP down(gelu(gate(x)) * up(x)) with the middle fused (modules.py:170-189): rotate + quantize, product,
    middle (tcq_mid2, or postg + pre2 with FUSE['split']), product, scale + rotate."""

    def __init__(self, gate_up, down):
        super().__init__()
        self.groups = [gate_up, down]
        self.gate_proj, self.up_proj, self.down_proj = KLinear(gate_up, 0), KLinear(gate_up, 1), KLinear(down, 0)

    def forward(self, x):
        gu, down = self.groups
        x2 = gu.prep(x)
        M, dev = x2.shape[0], x2.device
        if not FUSE['split'] and gu.spreads(M):
            z, b2 = gu.gated_down(gu.quantize(x2), down)
            STATS['fused_mlps'] += 1
            return down.posts(z, b2, x.shape)[0]
        acc, b = _first_half(gu, x)
        b2 = down.buffers(M, dev)
        s_tok, rs = (None, None) if acc.dtype == torch.float32 else (b['scale'], gu.rs)
        if FUSE['split']:
            g, u = (torch.empty(M, n, dtype=torch.bfloat16, device=dev) for n in gu.N)
            segs = [(acc, s.col0, None if rs is None else s.rs, s.sv, None, y, i == 0)
                    for i, (s, y) in enumerate(zip(gu.segments, (g, u)))]
            kernels.post_group(segs, acc.dtype, torch.bfloat16, s_tok, M, gelu_lut=kernels.gelu_table(dev))
            kernels.pre2(g, u, down.su, q=b2['q'], q4=b2['q4'], scale=b2['scale'])
        else:
            kernels.mid2(acc, s_tok, rs, gu.sv, down.su, q=b2['q'], q4=b2['q4'], scale=b2['scale'])
        STATS['fused_mlps'] += 1
        return down.posts(down.product(b2), b2, x.shape)[0]


class KPlainMLP(torch.nn.Module):
    """SigLIP MLP fc2(gelu(fc1(x))) with the middle fused (modules.py:192-206)."""

    def __init__(self, fc1, fc2):
        super().__init__()
        self.groups = [fc1, fc2]
        self.fc1, self.fc2 = KLinear(fc1, 0), KLinear(fc2, 0)

    def forward(self, x):
        first, second = self.groups
        acc, b = _first_half(first, x)
        b2 = second.buffers(acc.shape[0], acc.device)
        s_tok, rs = (None, None) if acc.dtype == torch.float32 else (b['scale'], first.rs)
        kernels.mid1(acc, s_tok, rs, first.sv, first.bias, second.su, q=b2['q'], q4=b2['q4'], scale=b2['scale'])
        STATS['fused_mlps'] += 1
        return second.posts(second.product(b2), b2, x.shape)[0]


_DEFER = {'on': False}


@contextlib.contextmanager
def deferred_outputs():
    """Inside this context a chained decoder layer at one token may return its output row before it is computed: the next
    layer's q/k/v product computes it (the down epilogue + residual) as part of its prologue and writes it before anything
    later on the stream reads it. Only for callers that pass each layer's output straight to the next layer and read
    nothing in between (the decode loops of gemma.BackbonePolicy); a layer whose input is not that output completes the
    row first. The last layer of a stack always computes its own output."""
    old = _DEFER['on']
    _DEFER['on'] = True
    try:
        yield
    finally:
        _DEFER['on'] = old


class Deferred:
    """A decoder layer's output row left to the next layer: the down product's int32 K parts z, the token scale s, the
    down group's row scales and output signs, the residual input x3 and the output x4 (not yet written)."""

    def __init__(self, z, s, rs, sv, x3, x4):
        self.z, self.s, self.rs, self.sv, self.x3, self.x4 = z, s, rs, sv, x3, x4

    def prologue(self, x2, norm, su):
        """The layer prologue of the next q/k/v product: writes x4 (= x2, the next layer's input) and computes the INT8 row
        of fwht(RMSNorm(x4) * su)."""
        return kernels.prologue(self.z, self.s, self.rs, self.sv, self.x3, x2, norm.weight, norm.eps, su)

    def complete(self):
        """Writes the output row alone (tcq_post_add_norm_pre without the norm)."""
        kernels.post_add_norm_pre(self.z, self.s, self.rs, self.sv, None, self.x3, self.x4)


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
        """What the previous layer left for exactly this input (x as passed, x2 its 2-D view): the q/k/v input buffers it
        computed, a Deferred record (its output row still to be computed, by this layer's q/k/v product), or None. A
        Deferred record that does not match the input is completed here, so the previous layer's output is valid."""
        h, self._handoff = self._handoff, None
        if h is None:
            return None
        xo, ver, ret, b = h
        if x2.data_ptr() != xo.data_ptr() or x2.shape != xo.shape or x2.dtype != xo.dtype:
            match = False
        elif ver is None:
            match = x is ret
        else:
            match = not x2.is_inference() and x2._version == ver
        if match:
            return b
        if isinstance(b, Deferred):
            b.complete()
        return None

    def _defers(self, M, z4, dn, nxt):
        """Whether this layer may leave its output row to the next layer's q/k/v product (inside deferred_outputs() only):
        one token, int32 sums of a two-sided down projection without bias, 2048-wide rows, a q/k/v group that takes the
        layer prologue (tcq_gemm_*_pro)."""
        nq = nxt.groups[0]
        return (_DEFER['on'] and FUSE['defer'] and M == 1 and z4.dtype == torch.int32 and dn.bias is None and not dn.one_sided
                and dn.Ntot == 2048 and nq.K == 2048 and nq.a8 and nq.col_scale is None)

    @staticmethod
    def _prologue_fits(z, og, gu):
        """Whether the o epilogue + residual + norm2 + rotate + quantize can run as the prologue of the gate | up product
        (tcq_gemm_tcq_pro): one token, int32 sums, a two-sided o projection without bias, 2048-wide rows, and a gate | up
        group on the spread middle (256 workgroups, one per CU, so each CU runs the prologue once). Measured on MI355X at
        one token: fly 18.1 -> 17.2 us for the two launches' work; on the resident plan's 1024 workgroups the prologue
        runs four times per CU and the pair gets slower (1.50 -> 1.72 ms per decode token), so it is not used there."""
        return (FUSE['prologue'] and z.dtype == torch.int32 and z.shape[-2] == 1 and og.bias is None and not og.one_sided
                and og.Ntot == 2048 and gu.K == 2048 and gu.a8 and gu.spreads(1))

    def _attn_prologue_fits(self, M, q, og):
        """Whether the attention's merge + o rotate + quantize can run as the prologue of the o product (tcq_gemm_*_pro with
        part): one token, a device attention with the split entry, 8 heads of 256 (2048-wide o input), plain signs. q: the
        BF16 query rows (None: the device attention is taken as given)."""
        a = self.self_attn
        return (FUSE['attn_prologue'] and M == 1 and hasattr(a, 'core_parts') and (q is None or a._device(q))
                and getattr(a, 'heads', 0) == 8 and getattr(a, 'head_dim', 0) == 256
                and og.K == 2048 and og.a8 and og.col_scale is None and og.k_parts(M) <= 2)

    def _attn_post_fits(self, M, z1, qkv, og, cache_k, cache_v):
        """Whether the q/k/v epilogue can run inside the attention's launch as well (tcq_attend_post_parts), with the merge in
        the o product's prologue: the attention prologue's conditions, FP32 z of a two-sided q | k | v group of widths
        2048, 256, 256 without biases, and a contiguous BF16 cache."""
        if not (FUSE['attn_post'] and z1.is_cuda and z1.dtype == torch.float32 and z1.dim() == 2 and z1.is_contiguous()
                and self._attn_prologue_fits(M, None, og) and not qkv.one_sided):
            return False
        segs = qkv.segments
        if [s.width for s in segs] != [2048, 256, 256] or any(s.bias is not None for s in segs):
            return False
        return all(c is None or (c.dtype == torch.bfloat16 and c.is_contiguous() and c.dim() == 2 and c.shape[-1] == 256)
                   for c in (cache_k, cache_v))

    @staticmethod
    def _unscaled(acc, b, group):
        """(token scales, row scales) the epilogue applies to acc: none for FP32 z, else the quantizer's and the group's."""
        return (None, None) if acc.dtype == torch.float32 else (b['scale'], group.rs)

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
        if isinstance(b, Deferred):
            # the previous layer's down epilogue + residual (writing this layer's input x2) + norm1 + rotate + quantize run
            # inside the q/k/v product's launch
            z1 = qkv.product(None, pro=b.prologue(x2, n1, qkv.su))
            b = None
            STATS['deferred_outputs'] += 1
        else:
            if b is None:
                b = qkv.buffers(M, dev)
                kernels.norm_pre(x2, n1.weight, n1.eps, qkv.su, q=b['q'], q4=b['q4'], scale=b['scale'])
            else:
                STATS['chained_prologues'] += 1
            z1 = qkv.product(b)
        if self._attn_post_fits(M, z1, qkv, og, cache_k, cache_v):
            # one token: the q/k/v epilogue runs inside the attention's launch (the query row never leaves it; the new key /
            # value rows go to kv_out), the chunk merge + o rotate + quantize inside the o product's launch
            a = self.self_attn
            kn, vn = kv_out if kv_out is not None else [torch.empty(M, s.width, dtype=torch.bfloat16, device=dev)
                                                        for s in qkv.segments[1:]]
            parts = kernels.attend_post_parts(z1, [(s.col0, s.sv) for s in qkv.segments], cache_k, cache_v, kn, vn, a.heads,
                                              causal_offset)
            k, v = kn.reshape(*shape[:-1], kn.shape[-1]), vn.reshape(*shape[:-1], vn.shape[-1])
            b2 = dict(q=None, q4=None, scale=torch.empty(M, dtype=torch.float32, device=dev))
            z = og.product(None, og.k_parts(M), pro=kernels.prologue_attn(parts, a.heads, og.su, scale=b2['scale']))
            STATS['attn_posts'] += 1
            STATS['attn_prologues'] += 1
        else:
            q, k, v = qkv.posts(z1, b, x2.shape, outs=None if kv_out is None else [None, kv_out[0], kv_out[1]])
            if self._attn_prologue_fits(M, q, og):
                # one token: the attention's chunk merge + o rotate + quantize run inside the o product's launch
                parts = self.self_attn.core_parts(q, k, v, cache_k, cache_v, causal_offset)
                b2 = dict(q=None, q4=None, scale=torch.empty(M, dtype=torch.float32, device=dev))
                z = og.product(None, og.k_parts(M), pro=kernels.prologue_attn(parts, self.self_attn.heads, og.su, scale=b2['scale']))
                STATS['attn_prologues'] += 1
            else:
                if hasattr(self.self_attn, 'core_quantized') and self.self_attn._device(q):
                    b2 = og.buffers(M, dev)
                    self.self_attn.core_quantized(q, k, v, cache_k, cache_v, causal_offset, og.su, b2['q'], b2['scale'],
                                                  q4=b2['q4'])
                else:
                    b2 = og.quantize(og.prep(self.self_attn.core(q, k, v, cache_k, cache_v, causal_offset)))
                z = og.product(b2, og.k_parts(M))
        x3 = torch.empty_like(x2)
        if self._prologue_fits(z, og, gu):
            # one token: the o epilogue + residual + norm2 + rotate + quantize run inside the gate | up product's launch
            pro = kernels.prologue(z, b2['scale'], og.rs, og.sv, x2, x3, n2.weight, n2.eps, gu.su)
            z4, b4 = gu.gated_down(None, dn, dn.k_parts(M), pro=pro)
            STATS['layer_prologues'] += 1
        else:
            b3 = gu.buffers(M, dev)
            kernels.post_add_norm_pre(z, *self._unscaled(z, b2, og), og.sv, og.bias, x2, x3, n2.weight, n2.eps, gu.su, q=b3['q'],
                                      q4=b3['q4'], scale=b3['scale'])
            z4, b4 = gu.gated_down(b3, dn, dn.k_parts(M))
        x4 = torch.empty_like(x2)
        nxt = self._next[0] if (self._next and FUSE['chain']) else None
        if nxt is None:
            kernels.post_add_norm_pre(z4, *self._unscaled(z4, b4, dn), dn.sv, dn.bias, x3, x4)
        elif self._defers(M, z4, dn, nxt):
            bn = Deferred(z4, b4['scale'], dn.rs, dn.sv, x3, x4)        # x4 is written by the next layer's q/k/v product
        else:
            nq, nn1 = nxt.groups[0], nxt.input_layernorm
            bn = nq.buffers(M, dev)
            kernels.post_add_norm_pre(z4, *self._unscaled(z4, b4, dn), dn.sv, dn.bias, x3, x4, nn1.weight, nn1.eps, nq.su,
                                      q=bn['q'], q4=bn['q4'], scale=bn['scale'])
        out = x4.reshape(shape)
        if nxt is not None:
            nxt._handoff = (x4, None if x4.is_inference() else x4._version, out, bn)
        STATS['fused_layers'] += 1
        return out, k, v


class RefLinear(torch.nn.Module):
    """The layer by definition, one unfused step per launch (modules.py:209-219 runs tcq_format.reference_linear):
    a8 / INT8 table: h = fwht(x * su) in FP32 -> per-token INT8 -> exact int32 product with the decoded INT8 weight ->
    (acc * s) * rs -> fwht -> * sv (+ bias) -> BF16. a8 / FP16 table: the INT8 activations times the FP16-table weight in
    FP64, then (z * s) * row scale. a8=False: the FP32 rotated activations times the decoded weight of `table` in FP64,
    * row scale, then the same output rotation (tcq_format.py:130-148). resident=False decodes on every call. GR00T records: a
    column scale joins the rotate + quantize launch (tcq_pre_cs); a one-sided layer skips the output rotation."""

    def __init__(self, layer, a8=True, table='int8', resident=True):
        super().__init__()
        if table not in ('int8', 'fp16'):
            raise ValueError('RefLinear: table is int8 or fp16')
        if layer.col_scale is not None and not a8:
            raise NotImplementedError('RefLinear: column scales are applied to quantized activations only')
        self.layer, self.a8, self.table, self.resident = [layer], a8, table, resident
        self.w8 = layer.w8_reference() if (table == 'int8' and resident) else None
        self.in_features, self.out_features, self.layer_name = layer.n, layer.m, layer.name
        self.register_buffer('weight', torch.empty(0, dtype=torch.bfloat16, device=layer.su.device), persistent=False)

    def forward(self, x):
        (L,) = self.layer
        shape = x.shape
        x2 = x.reshape(-1, L.n).contiguous()
        if x2.dtype not in (torch.bfloat16, torch.float32, torch.float16):
            x2 = x2.float()
        M, dev = x2.shape[0], x2.device
        y = torch.empty(M, L.m, dtype=torch.bfloat16, device=dev)
        if self.a8:
            q = torch.empty(M, L.n, dtype=torch.int8, device=dev)
            s = torch.empty(M, dtype=torch.float32, device=dev)
            if L.col_scale is None:
                h = kernels.rht(x2, L.su, torch.empty(M, L.n, dtype=torch.float32, device=dev))
                kernels.quantize_rows(h, q, s)
            else:
                kernels.pre(x2, L.su, q=q, scale=s, col_scale=L.col_scale)
            if self.table == 'int8':
                w8 = self.w8 if self.w8 is not None else L.w8_reference()
                acc = kernels.gemm_i8(q, w8, torch.empty(M, L.m, dtype=torch.int32, device=dev))
                kernels.post(acc, s, L.rs, L.sv, L.bias, y)
            else:                                           # INT8 activations times the FP16-table weights, FP64 sums
                z = (q.double() @ L.decode_f16().double().t()).float() * s[:, None] * L.row_scale.float()[None, :]
                kernels.post(z.contiguous(), None, None, L.sv, L.bias, y)
        else:
            h = kernels.rht(x2, L.su, torch.empty(M, L.n, dtype=torch.float32, device=dev))
            w = (self.w8 if self.w8 is not None else L.w8_reference()) if self.table == 'int8' else L.decode_f16()
            r = L.rs if self.table == 'int8' else L.row_scale.float()
            z = ((h.double() @ w.double().t()).float() * r[None, :]).contiguous()
            kernels.post(z, None, None, L.sv, L.bias, y)
        return y.reshape(*shape[:-1], L.m)


# ------------------------------------------------------------------------------------------------------- install
def set_submodule(model, name, module):
    parent, _, leaf = name.rpartition('.')
    setattr(model.get_submodule(parent) if parent else model, leaf, module)


def _norm_tensors(f):
    """(parameter name path, attribute, key) of the fine-tuned norm entries norm::<module>::<attr> of a dense file."""
    for key in sorted(f.keys()):
        kind, _, rest = key.partition('::')
        if kind == 'norm':
            module, _, attr = rest.partition('::')
            yield module, attr, key


def apply_row_state(model, row):
    """The fine-tuned norm weights stored beside the packed file (dense.safetensors entries norm::<module>::<attr>,
    modules.py:227-243). The reference's row-INT8 token embedding belongs to its private policy loader and is not applied."""
    path = F.packed_path(row).with_name('dense.safetensors')
    if not path.exists():
        return 0
    from safetensors import safe_open
    count = 0
    with safe_open(str(path), framework='pt', device='cpu') as f:
        for module, attr, key in _norm_tensors(f):
            target, value = getattr(model.get_submodule(module), attr), f.get_tensor(key)
            if (value.shape, value.dtype) != (target.shape, target.dtype):
                raise ValueError(f'{key}: {tuple(value.shape)} {value.dtype} does not match {tuple(target.shape)} {target.dtype}')
            target.data.copy_(value)
            count += 1
    return count


def plan_groups(names, layers, families=GROUPS):
    """Partition layer names into groups: the members of one family (of GROUPS by default) under one parent module form a
    group when the whole family is there and reads one input (_shares_input); every other layer is a group of its own.
    Groups come in the order of their first member."""
    buckets = {}
    for name in names:
        parent, _, leaf = name.rpartition('.')
        family = next((fam for fam in families if leaf in fam), None)
        buckets.setdefault((parent, family) if family else (name, None), {})[leaf] = name
    plan = []
    for (_, family), members in buckets.items():
        whole = family is not None and set(members) == set(family)
        if whole and _shares_input([layers[members[leaf]] for leaf in family]):
            plan.append([members[leaf] for leaf in family])
        else:
            plan.extend([n] for n in members.values())
    return plan


def _mode_of(runtime, streamed):
    if runtime == 'resident':
        return 'resident'
    return 'fly' if (runtime == 'fly' or streamed) else 'chunk'


def _fuse_mlps(model, heads):
    """Replace GemmaMLP / SiglipMLP modules whose layers are grouped (heads: first member name -> group) by the fused
    modules. Returns the count."""
    fused = 0
    for path, mod in list(model.named_modules()):
        kind = type(mod).__name__
        if kind == 'GemmaMLP':
            gu, dn = heads.get(f'{path}.gate_proj'), heads.get(f'{path}.down_proj')
            if gu is not None and len(gu.layers) == 2 and dn is not None and not gu.one_sided:
                set_submodule(model, path, KGatedMLP(gu, dn))
                fused += 1
        elif kind == 'SiglipMLP':
            f1, f2 = heads.get(f'{path}.fc1'), heads.get(f'{path}.fc2')
            if f1 is not None and f2 is not None and not f1.one_sided:
                set_submodule(model, path, KPlainMLP(f1, f2))
                fused += 1
    return fused


def _fuse_decoder_layers(model, heads):
    """Replace GemmaDecoderLayer modules whose attention projections are grouped and whose MLP is fused by
    KDecoderLayer, then link consecutive fused layers of each stack. Returns the count."""
    fused = 0
    for path, mod in list(model.named_modules()):
        if type(mod).__name__ != 'GemmaDecoderLayer':
            continue
        attn = f'{path}.self_attn'
        qkv, og = heads.get(f'{attn}.q_proj'), heads.get(f'{attn}.o_proj')
        if (qkv is None or len(qkv.layers) != 3 or og is None or not isinstance(getattr(mod, 'mlp', None), KGatedMLP)
                or not hasattr(mod.self_attn, 'core')):
            continue
        set_submodule(model, path, KDecoderLayer(mod, qkv, og, mod.mlp))
        fused += 1
    for stack in model.modules():
        if isinstance(stack, torch.nn.ModuleList):
            for a, b in zip(stack[:-1], stack[1:]):
                if isinstance(a, KDecoderLayer) and isinstance(b, KDecoderLayer):
                    a._next = [b]
    return fused


def install(policy, row=F.ROW, runtime='resident', a8=True, table='int8', reference_resident=True, layers=None):
    """Swap every quantizable nn.Linear of policy (or policy._model) found in the packed file of `row` (modules.py:246-311).
    layers: an already loaded {name: Layer} to use instead of reading the file."""
    if runtime not in RUNTIMES:
        raise ValueError(f'runtime {runtime!r} not in {RUNTIMES}')
    model = getattr(policy, '_model', policy)
    rule = rule_for(model)
    mods = dict(model.named_modules())
    if layers is None:
        stored = set(F.layer_names(row))
        names = [n for n, m in mods.items() if n in stored and rule.quantizable(n, m)]
    else:
        names = list(layers)
    for name in names:
        if not isinstance(mods.get(name), torch.nn.Linear):
            raise TypeError(f'{name}: {type(mods.get(name)).__name__} is not an nn.Linear')
    # biases live in the model; a module on the meta device carries none (the layer keeps its own, if any)
    biases = {n: mods[n].bias.detach().float().clone() for n in names
              if mods[n].bias is not None and not mods[n].bias.is_meta}
    info = dict(row=str(row), runtime=runtime, layers=len(names), policy=rule.name,
                norm_tensors=apply_row_state(model, row) if layers is None else 0)
    if layers is None:
        layers = F.load(row, device=next(model.parameters()).device, names=names, biases=biases)
    else:
        for n, b in biases.items():
            if layers[n].bias is None:
                layers[n].bias = b.to(layers[n].su.device).contiguous()
    if runtime == 'dense':
        for name in names:
            w = layers[name].dense(table)
            if mods[name].weight.shape != w.shape:
                raise ValueError(f'{name}: weight {tuple(mods[name].weight.shape)} != {tuple(w.shape)}')
            mods[name].weight.data.copy_(w.to(mods[name].weight.dtype))
        return info
    if runtime == 'reference':
        for name in names:
            set_submodule(model, name, RefLinear(layers[name], a8=a8, table=table, resident=reference_resident))
        return info
    groups = []
    for members in plan_groups(names, layers, rule.families):
        part = rule.part(members[0])
        group = Group([layers[n] for n in members], part, _mode_of(runtime, rule.streamed(part)), a8=a8)
        for i, n in enumerate(members):
            set_submodule(model, n, KLinear(group, i))
        if group.mode == 'resident':                        # the stream is not needed after load
            for L in group.layers:
                L.bits_resident, L.bits, L._words = False, None, None
        groups.append(group)
    heads = {g.layers[0].name: g for g in groups}
    fused = _fuse_mlps(model, heads) if (a8 and FUSE['mlp']) else 0
    fused_layers = _fuse_decoder_layers(model, heads) if (a8 and FUSE['mlp'] and FUSE['layer']) else 0
    torch.cuda.synchronize()
    policy._tcq_groups = groups
    modes = Counter(g.mode for g in groups)
    info.update(fused_layers=fused_layers, fused_mlps=fused, groups=len(groups),
                shared_rotations=sum(len(g.layers) for g in groups) - len(groups),
                modes={m: modes.get(m, 0) for m in ('resident', 'fly', 'chunk')},
                parts=dict(Counter(rule.part(n) for n in names)))
    return info


def decode_chunk(policy):
    """Operating point (iii): decode the action-generating part's layers once per action chunk, before the first denoising
    step (modules.py:314-320). Returns the number of layers decoded."""
    chunked = [g for g in getattr(policy, '_tcq_groups', ()) if g.mode == 'chunk']
    for g in chunked:
        g.decode()
    return sum(len(g.layers) for g in chunked)
