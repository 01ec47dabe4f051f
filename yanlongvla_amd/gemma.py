"""Gemma-shaped decoder stacks carrying the pi0.5 policy's module names, so that modules.install finds and swaps their
quantized Linear layers exactly as in the policy (baselines/common.py:51-58 names; GemmaMLP class name asserted by install,
modules.py:299-300). They drive the deploy path at the policy's shapes with synthetic weights. Between the quantized
Linears, RMSNorm and attention of BF16 device tensors run on this library's kernels (tcq_rmsnorm, tcq_attend), and the
residual adds, GELU and products of the unfused MLP are PyTorch; host tensors (CPU twins in tests) take the same formulas
in PyTorch.

  ExpertPolicy: the action expert (Gemma-300M-style: width 1024, MLP 4096 GeGLU, 8 query heads / 1 KV head of dim 256),
      action tokens attend to a fixed prefix KV cache and to each other; `sample_chunk` runs the flow-matching Euler steps.
  BackbonePolicy: the PaliGemma language model (width 2048, MLP 16384): causal prefill over the prefix, then single-token
      decode steps against the growing KV cache.
The norms are plain RMSNorm (the expert's AdaRMS time conditioning is outside the quantized path). Attention is computed in
FP32 with contiguous operands.
"""
import math

import torch
from torch import nn


class GemmaRMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(dim))

    def forward(self, x):
        if x.is_cuda and x.dtype == torch.bfloat16 and self.weight.dtype == torch.bfloat16:
            from . import kernels
            x2 = x.reshape(-1, x.shape[-1]).contiguous()
            return kernels.rmsnorm(x2, self.weight, self.eps, torch.empty_like(x2)).reshape(x.shape)
        xf = x.float()                  # host tensors (CPU twins of a model in tests): the same formula in PyTorch
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * (1.0 + self.weight.float())
        return y.to(x.dtype)


class GemmaMLP(nn.Module):
    def __init__(self, width, hidden):
        super().__init__()
        self.gate_proj = nn.Linear(width, hidden, bias=False)
        self.up_proj = nn.Linear(width, hidden, bias=False)
        self.down_proj = nn.Linear(hidden, width, bias=False)

    def forward(self, x):
        return self.down_proj(nn.functional.gelu(self.gate_proj(x), approximate='tanh') * self.up_proj(x))


def attend(q, k, v, heads, causal_offset=None):
    """softmax(q k^T / sqrt(d)) v for `heads` query heads sharing one KV head. q (M, heads*d), k / v (T, d) -> (M, heads*d),
    FP32 with contiguous operands. causal_offset: query i sees keys 0 .. causal_offset + i (None: all keys)."""
    M, d = q.shape[0], k.shape[1]
    qh = q.float().reshape(M, heads, d).transpose(0, 1).reshape(heads * M, d).contiguous()
    kt = k.float().t().contiguous()
    s = (qh @ kt) * (1.0 / math.sqrt(d))
    if causal_offset is not None:
        T = k.shape[0]
        i = torch.arange(M, device=q.device).repeat(heads)[:, None]
        j = torch.arange(T, device=q.device)[None, :]
        s = s.masked_fill(j > i + causal_offset, float('-inf'))
    p = torch.softmax(s, dim=-1)
    o = p @ v.float().contiguous()
    return o.reshape(heads, M, d).transpose(0, 1).reshape(M, heads * d)


class GemmaAttention(nn.Module):
    def __init__(self, width, heads, head_dim):
        super().__init__()
        self.heads, self.head_dim = heads, head_dim
        self.q_proj = nn.Linear(width, heads * head_dim, bias=False)
        self.k_proj = nn.Linear(width, head_dim, bias=False)
        self.v_proj = nn.Linear(width, head_dim, bias=False)
        self.o_proj = nn.Linear(heads * head_dim, width, bias=False)

    def _device(self, q):
        return q.is_cuda and q.dtype == torch.bfloat16 and self.head_dim == 256 and self.heads <= 8

    def core(self, q, k, v, cache_k=None, cache_v=None, causal_offset=None):
        """Attention of the projected q / k / v (the cache rows, if any, before this call's own keys / values). Device
        BF16 tensors go to the HIP attention kernel; host tensors (CPU twins in tests) to the same formula in PyTorch."""
        if self._device(q):
            from . import kernels
            o = torch.empty(q.shape[0], self.heads * self.head_dim, dtype=torch.bfloat16, device=q.device)
            return kernels.attend(q.contiguous(), cache_k, cache_v, k.contiguous(), v.contiguous(), self.heads, causal_offset, o=o)
        kk = k if cache_k is None else torch.cat([cache_k, k.to(cache_k.dtype)], 0)
        vv = v if cache_v is None else torch.cat([cache_v, v.to(cache_v.dtype)], 0)
        return attend(q, kk, vv, self.heads, causal_offset).to(q.dtype)

    def core_quantized(self, q, k, v, cache_k, cache_v, causal_offset, su, q8, scale, q4=None):
        """core followed by the rotate + quantize prologue of o_proj (signs su) in the same launches: q8 (row-major) and / or
        q4 (token blocks) and scale of the BF16 attention output, which itself is not stored. Device tensors only."""
        from . import kernels
        kernels.attend(q.contiguous(), cache_k, cache_v, k.contiguous(), v.contiguous(), self.heads, causal_offset, su=su,
                       q8=q8, scale=scale, q4=q4)

    def core_parts(self, q, k, v, cache_k, cache_v, causal_offset):
        """The first half of core_quantized: the attention's chunk partials, merged later by the o_proj product's prologue
        (kernels.prologue_attn). Device tensors only."""
        from . import kernels
        return kernels.attend_parts(q.contiguous(), cache_k, cache_v, k.contiguous(), v.contiguous(), self.heads, causal_offset)

    def forward(self, x, cache_k=None, cache_v=None, causal_offset=None):
        """x (M, width) -> (o_proj output, this call's k, v)."""
        q, k, v = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        return self.o_proj(self.core(q, k, v, cache_k, cache_v, causal_offset)), k, v


class GemmaDecoderLayer(nn.Module):
    def __init__(self, width, hidden, heads, head_dim):
        super().__init__()
        self.input_layernorm = GemmaRMSNorm(width)
        self.self_attn = GemmaAttention(width, heads, head_dim)
        self.post_attention_layernorm = GemmaRMSNorm(width)
        self.mlp = GemmaMLP(width, hidden)

    def forward(self, x, cache_k=None, cache_v=None, causal_offset=None, kv_out=None):
        """kv_out: None, or (k, v) tensors this call's keys / values are copied into (then returned in their place)."""
        a, k, v = self.self_attn(self.input_layernorm(x), cache_k, cache_v, causal_offset)
        x = x + a
        if kv_out is not None:
            kv_out[0].copy_(k)
            kv_out[1].copy_(v)
            k, v = kv_out
        return x + self.mlp(self.post_attention_layernorm(x)), k, v


class GemmaStack(nn.Module):
    def __init__(self, layers, width, hidden, heads, head_dim):
        super().__init__()
        self.layers = nn.ModuleList(GemmaDecoderLayer(width, hidden, heads, head_dim) for _ in range(layers))
        self.norm = GemmaRMSNorm(width)


class _Node(nn.Module):
    pass


class KVCache:
    """Per-layer key / value rows of a decoder stack in buffers with room for `room` more rows: a decode step writes its
    row in place (the layers' kv_out) instead of concatenating the whole cache, so the rows already there are never
    copied again. rewind() returns to the rows given at construction (the prefill's)."""

    def __init__(self, ks, vs, room):
        self.base = self.length = ks[0].shape[0]
        cap = self.base + room
        self.k = [torch.empty(cap, k.shape[1], dtype=k.dtype, device=k.device) for k in ks]
        self.v = [torch.empty(cap, v.shape[1], dtype=v.dtype, device=v.device) for v in vs]
        for dst, src in zip(self.k + self.v, list(ks) + list(vs)):
            dst[:self.base].copy_(src)

    def rewind(self):
        self.length = self.base

    def rows(self, i):
        """Layer i's cache rows so far and the destination views of the next row: (k, v, (k_next, v_next))."""
        P = self.length
        if P >= self.k[i].shape[0]:
            raise RuntimeError(f'KV cache full ({P} rows)')
        return self.k[i][:P], self.v[i][:P], (self.k[i][P:P + 1], self.v[i][P:P + 1])


EXPERT = dict(layers=18, width=1024, hidden=4096, heads=8, head_dim=256, action_dim=32)
BACKBONE = dict(layers=18, width=2048, hidden=16384, heads=8, head_dim=256, vocab=257152)


class ExpertPolicy(nn.Module):
    """paligemma_with_expert.gemma_expert.model.layers.{i}.{self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj}."""

    def __init__(self, layers=18, width=1024, hidden=4096, heads=8, head_dim=256, action_dim=32):
        super().__init__()
        self.paligemma_with_expert = _Node()
        self.paligemma_with_expert.gemma_expert = _Node()
        self.paligemma_with_expert.gemma_expert.model = GemmaStack(layers, width, hidden, heads, head_dim)
        self.action_in_proj = nn.Linear(action_dim, width)
        self.action_out_proj = nn.Linear(width, action_dim)
        self.prefix_k = self.prefix_v = None

    @property
    def stack(self):
        return self.paligemma_with_expert.gemma_expert.model

    def set_prefix(self, ks, vs):
        """Per-layer prefix keys / values (T, head_dim), as the backbone's prefill leaves them."""
        self.prefix_k, self.prefix_v = list(ks), list(vs)

    def velocity(self, x_t):
        h = self.action_in_proj(x_t.to(self.action_in_proj.weight.dtype))
        for i, layer in enumerate(self.stack.layers):
            h, _, _ = layer(h, self.prefix_k[i], self.prefix_v[i])
        return self.action_out_proj(self.stack.norm(h))

    def sample_chunk(self, noise, steps=10):
        """Flow matching from t = 1 to 0 with `steps` Euler steps: x <- x + dt v(x), dt = -1 / steps."""
        x, dt = noise, -1.0 / steps
        for _ in range(steps):
            x = x + dt * self.velocity(x).to(x.dtype)
        return x


class BackbonePolicy(nn.Module):
    """paligemma_with_expert.paligemma.language_model.layers.{i}...: prefill over prefix embeddings, then decode steps."""

    def __init__(self, layers=18, width=2048, hidden=16384, heads=8, head_dim=256, vocab=257152):
        super().__init__()
        self.paligemma_with_expert = _Node()
        self.paligemma_with_expert.paligemma = _Node()
        lm = GemmaStack(layers, width, hidden, heads, head_dim)
        self.paligemma_with_expert.paligemma.language_model = lm
        self.embed_tokens = nn.Embedding(vocab, width)
        self.width = width

    @property
    def stack(self):
        return self.paligemma_with_expert.paligemma.language_model

    def embed(self, ids):
        return (self.embed_tokens(ids) * math.sqrt(self.width)).to(self.embed_tokens.weight.dtype)

    def prefill(self, x):
        """x (T, width) prefix embeddings -> last hidden state, per-layer caches (k, v) of the T positions."""
        ks, vs = [], []
        h = x
        for layer in self.stack.layers:
            h, k, v = layer(h, causal_offset=0)
            ks.append(k)
            vs.append(v)
        return self.stack.norm(h), ks, vs

    def decode_step_cached(self, x, cache):
        """decode_step on a KVCache: the same hidden state, with this token's keys / values written into the cache."""
        from . import modules
        h = x
        with modules.deferred_outputs():                 # each layer's output goes straight to the next layer
            for i, layer in enumerate(self.stack.layers):
                ck, cv, out = cache.rows(i)
                h, _, _ = layer(h, ck, cv, kv_out=out)
        cache.length += 1
        return self.stack.norm(h)

    def decode_step(self, x, ks, vs):
        """One token x (1, width) against the caches; returns the hidden state and the caches grown by one row."""
        from . import modules
        h, nk, nv = x, [], []
        with modules.deferred_outputs():                 # each layer's output goes straight to the next layer
            for i, layer in enumerate(self.stack.layers):
                h, k, v = layer(h, ks[i], vs[i])
                nk.append(torch.cat([ks[i], k.to(ks[i].dtype)], 0))
                nv.append(torch.cat([vs[i], v.to(vs[i].dtype)], 0))
        return self.stack.norm(h), nk, nv


def synthetic_layers(model, seed, device, per_layer_scale=True):
    """Synthetic packed tensors for every quantizable Linear of model: uniform-random words, N(0, 1) FP16 tables, +-1 signs
    shared by the layers that read the same input (q/k/v; gate/up), FP16 scales in [0.5, 1.5]."""
    from . import modules
    from . import tcq_format as F
    g = torch.Generator(device=device).manual_seed(seed)
    out, su_of = {}, {}
    for name, mod in model.named_modules():
        if not modules.is_quantizable(name, mod):
            continue
        m, n = mod.out_features, mod.in_features
        parent, _, leaf = name.rpartition('.')
        share = next((grp for grp in modules.GROUPS if leaf in grp), None)
        key = (parent, share[0]) if share else name
        if key not in su_of:
            su_of[key] = (torch.randint(0, 2, (n,), generator=g, device=device) * 2 - 1).to(torch.int8)
        bits = torch.randint(-32768, 32768, ((m // 16) * (n // 16), 32), generator=g, device=device,
                             dtype=torch.int32).to(torch.int16)
        tlut = torch.randn(512, 2, generator=g, device=device).half()
        if per_layer_scale:
            row_scale = ((torch.rand(1, generator=g, device=device) + 0.5) * 0.05 / math.sqrt(n)).expand(m).half().contiguous()
        else:
            row_scale = ((torch.rand(m, generator=g, device=device) + 0.5) * 0.05 / math.sqrt(n)).half()
        sv = (torch.randint(0, 2, (m,), generator=g, device=device) * 2 - 1).to(torch.int8)
        out[name] = F.Layer(name, dict(bits=bits, tlut=tlut, row_scale=row_scale, su=su_of[key], sv=sv), device=device)
    return out


def make_policy(cls, device, seed=0, dtype=torch.bfloat16, **cfg):
    """A policy of class cls on device with every parameter allocated but the quantizable Linear weights left uninitialised
    (install replaces those modules): norms at their Gemma identity (weight 0), action projections / embeddings N(0, 1 / fan-in)."""
    from . import modules
    with torch.device('meta'):
        model = cls(**cfg)
    model = model.to_empty(device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, mod in model.named_modules():
            if isinstance(mod, GemmaRMSNorm):
                mod.weight.zero_()
            elif isinstance(mod, nn.Linear) and not modules.is_quantizable(name, mod):
                mod.weight.normal_(0.0, 1.0 / math.sqrt(mod.in_features), generator=g)
                if mod.bias is not None:
                    mod.bias.zero_()
            elif isinstance(mod, nn.Embedding):
                mod.weight.normal_(0.0, 1.0 / math.sqrt(mod.embedding_dim), generator=g)
    return model.to(dtype).requires_grad_(False)
