"""GR00T N1.7 module skeleton: the policy's Linear layer names and shapes (the quantization candidates of the released
checkpoint, 466 Linear, of which the GR00T rule quantizes 432: baselines/groot/groot_common.py:33-42), on the meta device,
so that modules.install finds and swaps them exactly as in the policy. It has no forward: it drives install and the
per-layer products at the policy's shapes.

  backbone  Qwen3-VL vision tower: 24 blocks {attn.qkv 3072x1024, attn.proj 1024x1024, mlp.linear_fc1 4096x1024,
            mlp.linear_fc2 1024x4096}, merger + 3 deepstack mergers {linear_fc1 4096x4096, linear_fc2 2048x4096};
            language model layers 0-15 {q 2048x2048, k / v 1024x2048, o 2048x2048, gate / up 6144x2048, down 2048x6144}
  head      vl_self_attention: 4 blocks {attn1.to_q / to_k / to_v / to_out.0 2048x2048, ff.net.0.proj 8192x2048,
            ff.net.2 2048x8192}; DiT: 32 blocks {attn1.to_q / to_out.0 1536x1536, attn1.to_k / to_v 1536x2048 in the even
            (cross-attention) blocks and 1536x1536 in the odd (self-attention) ones, ff.net.0.proj 6144x1536, ff.net.2
            1536x6144, norm1.linear 3072x1536 (AdaLN, dense)}; proj_out_1 3072x1536 and proj_out_2 1024x1536 (dense)
"""
import torch
from torch import nn

QUANTIZED_LAYERS = 432
QUANTIZED_PARAMETERS = 2_340_421_632      # the rule's total (groot_common.py:42)


class _Node(nn.Module):
    pass


def _linear(n_in, n_out, bias=True):
    return nn.Linear(n_in, n_out, bias=bias, device='meta')


def _attention(width, kv_in, names, out_name):
    a = _Node()
    q, k, v = names
    setattr(a, q, _linear(width, width))
    setattr(a, k, _linear(kv_in, width))
    setattr(a, v, _linear(kv_in, width))
    if out_name == 'to_out':
        a.to_out = nn.ModuleList([_linear(width, width)])
    else:
        setattr(a, out_name, _linear(width, width))
    return a


def _ff(width, hidden):
    ff = _Node()
    ff.net = nn.ModuleList([_Node(), nn.Identity(), _linear(hidden, width)])
    ff.net[0].proj = _linear(width, hidden)
    return ff


def _dit_block(width, cross_in, cross):
    b = _Node()
    b.norm1 = _Node()
    b.norm1.linear = _linear(width, 2 * width)
    b.attn1 = _attention(width, cross_in if cross else width, ('to_q', 'to_k', 'to_v'), 'to_out')
    b.ff = _ff(width, 4 * width)
    return b


def skeleton():
    """The GR00T N1.7 Linear layers on the meta device under their policy names (no weights allocated)."""
    root = _Node()
    root.backbone = _Node()
    root.backbone.model = _Node()
    root.backbone.model.model = _Node()
    visual = root.backbone.model.model.visual = _Node()
    visual.blocks = nn.ModuleList()
    for _ in range(24):
        blk = _Node()
        blk.attn = _Node()
        blk.attn.qkv = _linear(1024, 3072)
        blk.attn.proj = _linear(1024, 1024)
        blk.mlp = _Node()
        blk.mlp.linear_fc1 = _linear(1024, 4096)
        blk.mlp.linear_fc2 = _linear(4096, 1024)
        visual.blocks.append(blk)

    def merger():
        m = _Node()
        m.linear_fc1 = _linear(4096, 4096)
        m.linear_fc2 = _linear(4096, 2048)
        return m
    visual.merger = merger()
    visual.deepstack_merger_list = nn.ModuleList(merger() for _ in range(3))
    lm = root.backbone.model.model.language_model = _Node()
    lm.embed_tokens = nn.Embedding(151936, 2048, device='meta')
    lm.layers = nn.ModuleList()
    for _ in range(16):
        layer = _Node()
        layer.self_attn = _Node()
        layer.self_attn.q_proj = _linear(2048, 2048, bias=False)
        layer.self_attn.k_proj = _linear(2048, 1024, bias=False)
        layer.self_attn.v_proj = _linear(2048, 1024, bias=False)
        layer.self_attn.o_proj = _linear(2048, 2048, bias=False)
        layer.mlp = _Node()
        layer.mlp.gate_proj = _linear(2048, 6144, bias=False)
        layer.mlp.up_proj = _linear(2048, 6144, bias=False)
        layer.mlp.down_proj = _linear(6144, 2048, bias=False)
        lm.layers.append(layer)
    root.backbone.model.lm_head = _linear(2048, 151936, bias=False)
    head = root.action_head = _Node()
    head.vl_self_attention = _Node()
    head.vl_self_attention.transformer_blocks = nn.ModuleList()
    for _ in range(4):
        b = _Node()
        b.attn1 = _attention(2048, 2048, ('to_q', 'to_k', 'to_v'), 'to_out')
        b.ff = _ff(2048, 8192)
        head.vl_self_attention.transformer_blocks.append(b)
    head.model = _Node()
    head.model.transformer_blocks = nn.ModuleList(_dit_block(1536, 2048, cross=(i % 2 == 0)) for i in range(32))
    head.model.proj_out_1 = _linear(1536, 3072)
    head.model.proj_out_2 = _linear(1536, 1024)
    return root


def row_groups(m, n):
    """Row-group table count of the GR00T g16 records by layer size (groot_tcq.py:154-161): 16 tables from 8 M weights
    on, 8 from 4 M, 4 from 2 M, else 2; layers with fewer than 256 rows keep one table."""
    if m < 256:
        return 1
    w = m * n
    return 16 if w >= 8 << 20 else 8 if w >= 4 << 20 else 4 if w >= 2 << 20 else 2


def synthetic_layers(model, seed, device, one_sided=True, col_scale=True, tables=True, names=None):
    """Synthetic GR00T records for the quantizable layers of `model` (or the given names): uniform-random words, N(0, 1)
    FP16 row-group tables (row_groups; tables=False: one table), FP16 row scales, input signs and column scales shared by
    every layer of one input width (the signs of the GR00T bases depend on the width alone, groot_tcq.py:194-200),
    no output signs when one_sided (the 'tcq' base). Biases of the model's Linear layers are drawn too (N(0, 0.1))."""
    from . import modules
    from . import tcq_format as F
    g = torch.Generator(device=device).manual_seed(seed)
    by_width, out = {}, {}
    for name, mod in model.named_modules():
        if names is not None and name not in names:
            continue
        if names is None and not modules.groot_is_quantizable(name, mod):
            continue
        m, n = mod.out_features, mod.in_features
        if n not in by_width:
            su = (torch.randint(0, 2, (n,), generator=g, device=device) * 2 - 1).to(torch.int8)
            cs = (torch.rand(n, generator=g, device=device) + 0.5).half() if col_scale else None
            by_width[n] = (su, cs)
        su, cs = by_width[n]
        G = row_groups(m, n) if tables else 1
        t = dict(bits=torch.randint(-32768, 32768, ((m // 16) * (n // 16), 32), generator=g, device=device,
                                    dtype=torch.int32).to(torch.int16),
                 tlut=torch.randn(*((G,) if G > 1 else ()), 512, 2, generator=g, device=device).half(),
                 row_scale=((torch.rand(m, generator=g, device=device) + 0.5) * 0.02).half(), su=su)
        if not one_sided:
            t['sv'] = (torch.randint(0, 2, (m,), generator=g, device=device) * 2 - 1).to(torch.int8)
        if cs is not None:
            t['col_scale'] = cs
        bias = torch.randn(m, generator=g, device=device) * 0.1 if mod.bias is not None else None
        out[name] = F.Layer(name, t, bias=bias, device=device)
    return out
