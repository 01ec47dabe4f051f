"""CPU oracle of the TCQ W2A8 deploy path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import this module, and only as the
checker (or, for `cpu_baseline`, as the timed CPU restatement). The product package `yanlongvla_amd` never imports it.

It restates, in numpy on the CPU, the reference arithmetic of deploy/tcq_kernels/tcq_format.py (the definition the reference's
CUDA kernels are checked against bit for bit, deploy/tcq_kernels/parity.py:121-172) plus the rounding points of the fused
kernel chains in deploy/tcq_kernels/kernels.py. Every function cites the reference lines it follows.

Conventions
  * float32 arrays stand for FP32 tensors; BF16 values travel as uint16 bit patterns (`bf16_bits` / `bf16_to_f32`).
  * `bits` is the packed trellis stream, shape (m/16 * n/16, 32), the uint16 words of each 16 x 16 tile (int16 view allowed).

How each function is pinned (tests/test_oracle.py):
  block_widths, fwht, states_from_bits, lookup, snap, quantize_tokens, int_matmul, reference_linear, Layer.dense
      -> golden vectors written by importing the reference's own tcq_format.py (tests/golden/make_golden.py), bit-exact
         (reference_linear with a8=False: within 1e-6, its FP64 matmul sums in a different order), plus closed forms:
         dense Sylvester Hadamard (fwht), bit-by-bit window read of the u16 stream (states_from_bits), the state recurrence
         s[t+1] = ((s[t] << 4) | next nibble) & 0xffff with tail-biting, exact int64 products (int_matmul).
  gelu_tanh_bf16 -> PyTorch's own torch.nn.functional.gelu(approximate='tanh') (the library routine the reference tabulates).
  rmsnorm_bf16 -> PyTorch's own RMSNorm formula in FP64 (within one BF16 rounding; the summation order is the kernels').
  w2_linear -> golden vectors of the reference's reference_linear(a8=False, table='int8') on inputs whose rotated activations
         are BF16-exact integers (n = 256): the expert variant equals them bit for bit, also for inputs offset by less than
         half a BF16 ulp (its rounding of h); the prefill variant equals the exact integer product rounded by PyTorch's BF16
         cast and scaled (modules.py:120-130); planted slips (no rounding of h, accumulator rounded or rounded after the
         scale) fail (tests/test_oracle.py).
  mlp_middle, plain_middle, pre2, quantize_channels, w8a8_reference -> compositions of the pinned functions with the rounding
         points written in deploy/tcq_kernels/kernels.py:272-277, 303 (checked against the unfused chain in the tests).
"""
import math

import numpy as np

__all__ = ['block_widths', 'fwht', 'states_from_bits', 'lookup', 'snap', 'quantize_tokens', 'int_matmul', 'Layer',
           'reference_linear', 'bf16_bits', 'bf16_to_f32', 'gelu_tanh_bf16', 'mlp_middle', 'plain_middle', 'pre2', 'rmsnorm_bf16', 'w2_linear', 'quantize_channels',
           'w8a8_reference', 'q4_layout', 'random_layer']


# ------------------------------------------------------------------------------------------------------------ number formats
def bf16_bits(x):
    """float32 -> BF16 bit patterns, round to nearest even, NaN -> 0x7fc0 (c10::BFloat16; deploy/tcq_kernels/kernels.py:20-25)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7fffffff) > 0x7f800000
    r = ((u + 0x7fff + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7fc0
    return r


def bf16_to_f32(b):
    """BF16 bit patterns (uint16 / int16) -> float32 (exact)."""
    return (np.asarray(b).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------------------------------------------- rotations
def block_widths(width):
    """Binary decomposition of a width into descending powers of two (tcq_format.py:26-30)."""
    out = []
    while width:
        b = 1 << (width.bit_length() - 1)
        out.append(b)
        width -= b
    return out


def fwht(x):
    """Block Walsh on the last axis in FP32: radix-2 butterflies (a + b, a - b) in stage order h = 1, 2, 4, ..., then an FP32
    multiply by float32(1 / sqrt(w)) per block (tcq_format.py:44-55, constant tcq_format.py:36-41)."""
    x = np.asarray(x, dtype=np.float32)
    outs, off = [], 0
    for w in block_widths(x.shape[-1]):
        y, h = x[..., off:off + w], 1
        while h < w:
            y = y.reshape(*y.shape[:-1], w // (2 * h), 2, h)
            a, b = y[..., 0, :], y[..., 1, :]
            y = np.stack((a + b, a - b), axis=-2).reshape(*y.shape[:-3], w)
            h *= 2
        outs.append(y * np.float32(1.0 / math.sqrt(w)))
        off += w
    return np.concatenate(outs, -1) if len(outs) > 1 else outs[0]


# ------------------------------------------------------------------------------------------------------------------- decode
def states_from_bits(bits, m, n):
    """Windowed read (tcq_format.py:58-63): state t (0..127) of a tile = bits [4t, 4t + 16) of its 512-bit stream of 32 uint16
    words, most significant bit first, tail-biting; tile (I, J), row r, pair p <-> t = 8 r + p. -> (m, n/2) int64."""
    b = np.asarray(bits).astype(np.int64) & 0xffff
    t = np.arange(128)
    w, r = t // 4, t % 4
    st = (((b[:, w] << 16) | b[:, (w + 1) % 32]) >> (16 - 4 * r)) & 0xffff
    return st.reshape(m // 16, n // 16, 16, 8).transpose(0, 2, 1, 3).reshape(m, n // 2)


def lookup(states, table):
    """(m, n/2) states + (512, 2) table -> (m, n): x = (s + 1) s, value = table[(x >> 6) & 511], the first coordinate negated
    when bit 15 of x is set (tcq_format.py:66-71). A (G, 512, 2) table holds row-group tables: rows split evenly into G
    contiguous groups, row i reading table i // (m / G) (groot_tcq.py:154-175, decode_normalized)."""
    x = (states + 1) * states
    table = np.asarray(table)
    if table.ndim == 3:
        G, m = table.shape[0], states.shape[0]
        grp = (np.arange(m) // (m // G))[:, None]
        v = table[grp, (x >> 6) & 511]
    else:
        v = table[(x >> 6) & 511]
    v0 = np.where(((x >> 15) & 1).astype(bool), -v[..., 0], v[..., 0])
    return np.stack((v0, v[..., 1]), -1).reshape(states.shape[0], -1)


def snap(tlut, row_scale):
    """INT8 table and row scale (tcq_format.py:74-77). `127.0 / tensor` is Tensor.__rdiv__ = reciprocal() * 127, so the gain is
    float32(float32(1 / amax) * 127); t8 = clamp(round_half_even(tlut * g), +-127); rs = float32(row_scale) / g (true division)."""
    t = np.asarray(tlut).astype(np.float32)
    if t.ndim == 3:                       # row-group tables: each table snaps on its own, each row uses its group's gain
        G = t.shape[0]
        parts = [snap(t[i], np.asarray(row_scale).reshape(G, -1)[i]) for i in range(G)]
        return (np.stack([p[0] for p in parts]), np.concatenate([p[1] for p in parts]),
                np.array([p[2] for p in parts], dtype=np.float32))
    amax = np.float32(np.abs(t).max())
    g = np.float32(np.float32(1.0) / amax) * np.float32(127.0)
    t8 = np.clip(np.round(t * g), -127, 127).astype(np.int8)
    rs = np.asarray(row_scale).astype(np.float32) / g
    return t8, rs.astype(np.float32), np.float32(g)


# --------------------------------------------------------------------------------------------------------------- activations
def quantize_tokens(h):
    """Per-token symmetric INT8 (tcq_format.py:119-122): s = amax / 127 (FP32 true division), 1 for an all-zero row;
    q = clamp(round_half_even(h / s), +-127)."""
    h = np.asarray(h, dtype=np.float32)
    amax = np.abs(h).max(axis=1, keepdims=True)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.round(h / s), -127, 127).astype(np.int8)
    return q, s


def quantize_channels(w):
    """Per-output-channel symmetric INT8 of a dense (N, K) weight: the per-token rule of quantize_tokens applied to each row."""
    q, s = quantize_tokens(w)
    return q, s[:, 0]


def int_matmul(q, w8):
    """Exact (M, K) int8 x (N, K) int8 -> (M, N) int32 (tcq_format.py:110-116, CPU branch: FP64 product, exact since
    |acc| <= K * 127^2 < 2^53)."""
    return (np.asarray(q).astype(np.float64) @ np.asarray(w8).astype(np.float64).T).astype(np.int32)


def q4_layout(q):
    """(M, K) int8 -> (K/4, M) int32 words, 4 consecutive inputs per little-endian word, token = column (the small-M product
    layout, deploy/tcq_kernels/kernels.py:170-184 and parity.py:151)."""
    M, K = q.shape
    return np.ascontiguousarray(np.ascontiguousarray(q).view(np.int32).reshape(M, K // 4).T)


# ----------------------------------------------------------------------------------------------------------------- the layer
class Layer:
    """One quantized Linear (tcq_format.py:80-107): packed tensors + the derived INT8 table / row scale. Optional GR00T
    record fields (baselines/groot/simpler/main_row/scripts/groot_tcq.py:178-191): no 'sv' = a one-sided layer
    W = Q H_n S_u (no output rotation); 'col_scale' (n,) FP16 = diag(c) between Q and the input rotation."""

    def __init__(self, name, tensors, bias=None):
        self.name = name
        self.bits = np.asarray(tensors['bits']).astype(np.int16)
        self.tlut = np.asarray(tensors['tlut']).astype(np.float16)
        self.row_scale = np.asarray(tensors['row_scale']).astype(np.float16)
        self.su = np.asarray(tensors['su']).astype(np.int8)
        self.sv = np.asarray(tensors['sv']).astype(np.int8) if tensors.get('sv') is not None else None
        cs = tensors.get('col_scale')
        self.col_scale = None if cs is None else np.asarray(cs).astype(np.float16)
        self.m, self.n = self.row_scale.size, self.su.size
        assert self.bits.shape == ((self.m // 16) * (self.n // 16), 32) and self.m % 16 == 0 and self.n % 16 == 0, name
        self.t8, self.rs, self.gain = snap(self.tlut, self.row_scale)
        self.bias = None if bias is None else np.asarray(bias, dtype=np.float32)

    def states(self):
        return states_from_bits(self.bits, self.m, self.n)

    def w8_reference(self):
        return lookup(self.states(), self.t8.astype(np.int16)).astype(np.int8)

    def dense(self, table='fp16'):
        """Original-basis FP32 weight S_v H_m diag(r) Q diag(c) H_n S_u (tcq_format.py:100-107; groot_tcq.py:178-191 for
        the column scale c and the one-sided form without S_v H_m)."""
        if table == 'fp16':
            q = lookup(self.states(), self.tlut.astype(np.float32)) * self.row_scale.astype(np.float32)[:, None]
        else:
            q = self.w8_reference().astype(np.float32) * self.rs[:, None]
        if self.col_scale is not None:
            q = q * self.col_scale.astype(np.float32)[None, :]
        w = fwht(q) * self.su.astype(np.float32)[None, :]
        if self.sv is None:
            return w
        return (fwht(np.ascontiguousarray(w.T)) * self.sv.astype(np.float32)[None, :]).T


def reference_linear(x, layer, a8=True, table='int8', w8=None, out_dtype='bf16'):
    """The W2A8 layer definition (tcq_format.py:125-148). x: float32 array (..., n) (BF16 / FP16 inputs converted exactly).
    out_dtype: 'bf16' -> uint16 bit patterns, 'f32' -> float32, 'f16' -> float16."""
    x = np.asarray(x, dtype=np.float32)
    shape = x.shape
    h = fwht(x.reshape(-1, shape[-1]) * layer.su.astype(np.float32))
    if layer.col_scale is not None:              # GR00T column scale on the rotated activations (the weight's diag(c))
        h = h * layer.col_scale.astype(np.float32)
    if table == 'int8':
        w8 = layer.w8_reference() if w8 is None else w8
        if a8:
            q, s = quantize_tokens(h)
            z = (int_matmul(q, w8).astype(np.float32) * s) * layer.rs[None, :]
        else:
            z = (h.astype(np.float64) @ w8.astype(np.float64).T).astype(np.float32) * layer.rs[None, :]
    else:
        wq = lookup(layer.states(), layer.tlut.astype(np.float32))
        r = layer.row_scale.astype(np.float32)[None, :]
        if a8:
            q, s = quantize_tokens(h)
            z = ((q.astype(np.float64) @ wq.astype(np.float64).T).astype(np.float32) * s) * r
        else:
            z = (h.astype(np.float64) @ wq.astype(np.float64).T).astype(np.float32) * r
    y = z if layer.sv is None else fwht(z) * layer.sv.astype(np.float32)     # one-sided layers: no output rotation
    if layer.bias is not None:
        y = y + layer.bias
    y = y.reshape(*shape[:-1], -1)
    if out_dtype == 'bf16':
        return bf16_bits(y)
    if out_dtype == 'f16':
        return y.astype(np.float16)
    return y.astype(np.float32)


# ------------------------------------------------------------------------------------------------------------- fused chains
def gelu_tanh_bf16(b):
    """GELU (tanh approximation) of BF16 bit patterns -> BF16 bit patterns, by PyTorch's CPU routine
    torch.nn.functional.gelu(x, approximate='tanh') (what deploy/tcq_kernels/kernels.py:563-569 tabulates on the device)."""
    import torch
    t = torch.from_numpy(np.asarray(b).astype(np.int16)).view(torch.bfloat16)
    return torch.nn.functional.gelu(t, approximate='tanh').view(torch.int16).numpy().astype(np.uint16)


def post_bf16(z, sv, bias=None):
    """Scaled accumulator row -> block Walsh -> sign -> bias -> BF16 bits (deploy/tcq_kernels/kernels.py:221-230)."""
    y = fwht(z) * np.asarray(sv).astype(np.float32)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return bf16_bits(y)


def pre2(g_bits, u_bits, su):
    """x = BF16(g * u) -> sign -> block Walsh -> per-token INT8 (deploy/tcq_kernels/kernels.py:295-307)."""
    prod = bf16_to_f32(bf16_bits(bf16_to_f32(g_bits) * bf16_to_f32(u_bits)))
    return quantize_tokens(fwht(prod * np.asarray(su).astype(np.float32)))


def mlp_middle(z_gate, z_up, sv_gate, sv_up, su_down, gelu=gelu_tanh_bf16):
    """Gated-MLP middle on scaled FP32 accumulators (deploy/tcq_kernels/kernels.py:263-278): gate -> Walsh -> sign -> BF16 ->
    GELU; up -> Walsh -> sign -> BF16; BF16 product -> down-projection rotate + INT8. Returns (q, s, g_bits, u_bits)."""
    g = gelu(post_bf16(z_gate, sv_gate))
    u = post_bf16(z_up, sv_up)
    q, s = pre2(g, u, su_down)
    return q, s, g, u


def plain_middle(z, sv, bias, su, gelu=gelu_tanh_bf16):
    """Plain-MLP middle on a scaled FP32 accumulator (deploy/tcq_kernels/kernels.py:280-292): Walsh -> sign -> bias -> BF16 ->
    GELU -> sign flip of the next layer -> Walsh -> per-token INT8. Returns (q, s, g_bits)."""
    g = gelu(post_bf16(z, sv, bias))
    q, s = quantize_tokens(fwht(bf16_to_f32(g) * np.asarray(su).astype(np.float32)))
    return q, s, g


def w2_linear(x, layer, small):
    """W2 float path (deploy/tcq_kernels/modules.py:117-144; kernels.py:309-337, 442-489): h = BF16(fwht(x * su)), the
    INT8 table values as weights, FP32 accumulation. Expert (small): z = acc * rs in FP32. Prefill: acc rounded to BF16 (the
    BF16 result of the BF16 matmul), z = bf16(acc) * rs. Then fwht(z) * sv (+ bias) -> BF16 bits. The product is summed in
    FP64 here; a device's FP32 sums differ in the last bits."""
    x = np.asarray(x, dtype=np.float32)
    h = bf16_to_f32(bf16_bits(fwht(x.reshape(-1, layer.n) * layer.su.astype(np.float32))))
    acc = (h.astype(np.float64) @ layer.w8_reference().astype(np.float64).T).astype(np.float32)
    if not small:
        acc = bf16_to_f32(bf16_bits(acc))
    return post_bf16(acc * layer.rs[None, :], layer.sv, layer.bias)


def rmsnorm_bf16(x, w_bits, eps):
    """Gemma RMSNorm as the device kernels define it (the decoder layers' norm, fused into their prologues; not part of the
    reference's quantized path): y = bf16((x * r) * (1 + w)), r = 1 / sqrt(ss / K + eps) in FP32, ss summed as 16-element
    sequential chunk sums followed by a pairwise tree over the chunks (stride 1, 2, 4, ...). x float32 (M, K) of BF16 values,
    w_bits BF16 bit patterns (K,). Returns BF16 bit patterns."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    xs = x.reshape(M, K // 16, 16)
    a = np.zeros((M, K // 16), dtype=np.float32)
    for k in range(16):
        a = a + xs[:, :, k] * xs[:, :, k]
    C, h = K // 16, 1
    while h < C:
        j = np.arange(0, C - h, 2 * h)
        a[:, j] = a[:, j] + a[:, j + h]
        h *= 2
    r = np.float32(1.0) / np.sqrt(a[:, 0] / np.float32(K) + np.float32(eps))
    one_w = np.float32(1.0) + bf16_to_f32(w_bits)
    return bf16_bits((x * r[:, None]) * one_w[None, :])


def w8a8_reference(a, w):
    """W8A8 GEMM contract: per-token INT8 of a (M, K), per-channel INT8 of w (N, K), exact INT32 accumulators, then
    BF16((acc * s_token) * s_channel) -- the order of tcq_format.py:135."""
    qa, sa = quantize_tokens(a)
    qw, sw = quantize_channels(w)
    acc = int_matmul(qa, qw)
    y = (acc.astype(np.float32) * sa) * sw[None, :]
    return dict(qa=qa, sa=sa[:, 0], qw=qw, sw=sw, acc=acc, y=bf16_bits(y))


# ----------------------------------------------------------------------------------------------------------- synthetic layers
def random_layer(m, n, seed, name='layer', bias=False, scale_range=(0.5, 1.5), per_layer_scale=True, groups=1, one_sided=False,
                 col_scale=False):
    """Seeded synthetic layer: uniform-random packed words, N(0, 1) FP16 table (groups > 1: (G, 512, 2) row-group tables,
    table g scaled by 1 + g / 4), +-1 signs, FP16 scale drawn from scale_range (one per layer broadcast to all rows when
    per_layer_scale, else one per row). one_sided: no output signs (no output rotation); col_scale: FP16 column scales
    drawn from [0.5, 1.5]."""
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 16, size=((m // 16) * (n // 16), 32), dtype=np.uint32).astype(np.uint16).view(np.int16)
    tlut = rng.standard_normal((512, 2)).astype(np.float16)
    if groups > 1:
        tlut = np.stack([(rng.standard_normal((512, 2)) * (1 + g / 4)).astype(np.float16) for g in range(groups)])
    if per_layer_scale:
        row_scale = np.full(m, rng.uniform(*scale_range), dtype=np.float16)
    else:
        row_scale = rng.uniform(*scale_range, size=m).astype(np.float16)
    su = np.where(rng.integers(0, 2, n) > 0, 1, -1).astype(np.int8)
    sv = np.where(rng.integers(0, 2, m) > 0, 1, -1).astype(np.int8)
    b = rng.standard_normal(m).astype(np.float32) * np.float32(0.1) if bias else None
    t = dict(bits=bits, tlut=tlut, row_scale=row_scale, su=su, sv=None if one_sided else sv)
    if col_scale:
        t['col_scale'] = rng.uniform(0.5, 1.5, size=n).astype(np.float16)
    return Layer(name, t, bias=b)
