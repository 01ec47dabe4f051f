"""Op-level helpers over the HIP library: caller-allocated outputs, dtype dispatch on the tensor dtype, launches on the current
stream. Names and argument meaning follow the reference's launch helpers (deploy/tcq_kernels/kernels.py:572-696); the
functions added here (rht, pre_h16, quantize_rows, repack, decode_f16, gemv_f16, ...) have no reference counterpart and say so.
"""
import ctypes

import torch

from . import _lib
from ._lib import DTYPE, call, ptr, stream


def _dt(t, allowed, what):
    d = DTYPE.get(t.dtype)
    if d not in allowed:
        raise TypeError(f'{what}: unsupported dtype {t.dtype}')
    return d


def _contig(*ts):
    for t in ts:
        if t is not None and not t.is_contiguous():
            raise ValueError('tensors passed to the TCQ kernels must be contiguous')


# Token-block layout of INT8 activations (include/tcq_api.h): a (ceil(M / 16), K / 16, 16, 16) int8 tensor, element
# [b, g, r, c] = token 16 b + r, column 16 g + c. The quantizers write it through q4 (ldq = LDQ_TOKEN_BLOCKS) and the
# small-M products read it (out_dtype | Q_TOKEN_BLOCKS): every 16-token x 64-column activation fragment is one contiguous KiB.
LDQ_TOKEN_BLOCKS = -16
Q_TOKEN_BLOCKS = 0x100
# K parts of a small-M product (include/tcq_api.h): int32 sums over 2 or 4 consecutive ranges of the 256-column K chunks, part
# p at out + p * M * ldo; the fused epilogue post_add_norm_pre adds them. A product of few tile rows then fills the chip.
K_PARTS = {2: 0x200, 4: 0x400}


def token_blocks(M, K, device):
    """An uninitialised token-block activation buffer for M tokens of K columns (K % 16 == 0)."""
    return torch.empty((M + 15) // 16, K // 16, 16, 16, dtype=torch.int8, device=device)


def rows_of_token_blocks(tb, M):
    """The (M, K) row-major view of a token-block tensor (a copy)."""
    return tb.permute(0, 2, 1, 3).reshape(tb.shape[0] * 16, tb.shape[1] * 16)[:M]


# ------------------------------------------------------------------------------------------------------------- load time
def _groups(table):
    """Number of (512, 2) tables in a table tensor: (512, 2) -> 1, (G, 512, 2) -> G (row-group tables)."""
    n = table.numel()
    if n % 1024:
        raise ValueError(f'a table tensor holds whole (512, 2) tables, got {tuple(table.shape)}')
    return n // 1024


def snap(tlut, row_scale, t8=None, rs=None, gain=None):
    """INT8 table / row scale / gain of tcq_format.snap (reference tcq_format.py:74-77), computed on the device. A
    (G, 512, 2) row-group table snaps per group: t8 (G, 512, 2), gain (G,), rs of each row from its group's gain."""
    dev = tlut.device
    G = _groups(tlut)
    shape = (512, 2) if tlut.dim() == 2 else (G, 512, 2)
    t8 = torch.empty(*shape, dtype=torch.int8, device=dev) if t8 is None else t8
    rs = torch.empty(row_scale.numel(), dtype=torch.float32, device=dev) if rs is None else rs
    gain = torch.empty(G, dtype=torch.float32, device=dev) if gain is None else gain
    _contig(tlut, row_scale, t8, rs)
    call('tcq_snap_groups', ptr(tlut), G, ptr(row_scale), row_scale.numel(), ptr(t8), ptr(rs), ptr(gain), stream())
    return t8, rs, gain


def repack_words(m, n):
    return int(_lib.lib().tcq_repack_words(m, n))


def repack(bits, m, n, out=None):
    """Reference word layout -> device layout of the fused products (no reference counterpart; a load-time permutation)."""
    out = torch.empty(repack_words(m, n), dtype=torch.int32, device=bits.device) if out is None else out
    _contig(bits, out)
    call('tcq_repack', ptr(bits), ptr(out), m, n, stream())
    return out


# ---------------------------------------------------------------------------------------------------------------- decode
def decode(bits, t8, out):
    """Dense INT8 decode, out (m, n) int8 (reference kernels.py:653-656); t8 (512, 2) or (G, 512, 2) row-group tables."""
    m, n = out.shape
    _contig(bits, t8, out)
    call('tcq_decode_i8_groups', ptr(bits), ptr(t8), _groups(t8), ptr(out), m, n, stream())


def decode_words(words, t8, out):
    """decode from the tcq_repack words (one (512, 2) table): the same bytes, through the fused products' layout."""
    m, n = out.shape
    _contig(words, t8, out)
    call('tcq_decode_i8_words', ptr(words), ptr(t8), ptr(out), m, n, stream())


def decode_f16(bits, tlut, out):
    """Dense decode through the FP16 table, out (m, n) float16 (exact lookup(states, tlut))."""
    m, n = out.shape
    _contig(bits, tlut, out)
    call('tcq_decode_f16_groups', ptr(bits), ptr(tlut), _groups(tlut), ptr(out), m, n, stream())


def decode_bf16(bits, tb, out):
    """Dense decode through the BF16 bit patterns tb (512, 2) of the INT8 table values (the W2 float path), out (m, n)
    bfloat16 (reference kernels.decode_bf16, kernels.py:683-686)."""
    m, n = out.shape
    _contig(bits, tb, out)
    call('tcq_decode_f16_groups', ptr(bits), ptr(tb), _groups(tb), ptr(out), m, n, stream())


# -------------------------------------------------------------------------------------------------------------- rotation
def rht(x, su, y):
    """y = fwht(x * su) row by row (su may be None). x, y (M, n); dtypes float32 / bfloat16 / float16."""
    M, n = x.shape
    if y.shape != x.shape or (su is not None and su.numel() != n):
        raise ValueError(f'rht: y {tuple(y.shape)} / su must match x {tuple(x.shape)}')
    call('tcq_rht', ptr(x), _dt(x, (0, 1, 2), 'rht x'), x.stride(0), ptr(su), ptr(y), _dt(y, (0, 1, 2), 'rht y'), y.stride(0),
         M, n, stream())
    return y


def pre(x, su, q=None, q4=None, scale=None, col_scale=None):
    """x (M, K) BF16 / FP32 / FP16 contiguous -> q (M, K) int8 and / or q4 (K/4, ld) int32 or token blocks, scale (M,) FP32
    (reference kernels.py:602-606). col_scale: FP16 (K,) column scales of a GR00T record, applied to the rotated activations
    before they are quantized (tcq_pre_cs); not a reference argument."""
    M, K = x.shape
    _contig(x, su, q, q4, scale, col_scale)
    if col_scale is None:
        call('tcq_pre', ptr(x), _dt(x, (0, 1, 2), 'pre x'), ptr(su), ptr(q), ptr(q4), _ldq(q4), ptr(scale), M, K, stream())
        return
    if col_scale.dtype != torch.float16 or col_scale.numel() != K:
        raise ValueError(f'pre: col_scale must be ({K},) float16')
    call('tcq_pre_cs', ptr(x), _dt(x, (0, 1, 2), 'pre x'), ptr(su), ptr(col_scale), ptr(q), ptr(q4), _ldq(q4), ptr(scale), M, K,
         stream())


def pre_h16(x, su, h16, hscale):
    """Float path: h16 (M, K) float16 = fwht(x * su) / hscale, hscale (M,) FP32 powers of two."""
    M, K = x.shape
    _contig(x, su, h16, hscale)
    call('tcq_pre_h16', ptr(x), _dt(x, (0, 1, 2), 'pre_h16 x'), ptr(su), ptr(h16), ptr(hscale), M, K, stream())


def quantize_rows(x, q, scale):
    """Per-row symmetric INT8 without rotation (tcq_format.quantize_tokens): q (M, K) int8, scale (M,) FP32."""
    M, K = x.shape
    _contig(q, scale)
    call('tcq_quantize_rows', ptr(x), _dt(x, (0, 1, 2), 'quantize_rows x'), x.stride(0), ptr(q), ptr(scale), M, K, stream())


def post(acc, s, rs, sv, bias, y, col0=0):
    """acc (M, lda) int32 (scaled here by s, rs), FP32 (already scaled) or BF16 (scaled by rs); columns col0 .. col0 + N -> y
    (M, N) BF16 / FP16 / FP32 (reference kernels.py:612-615). sv None: a one-sided layer, no output rotation."""
    M, N = y.shape
    _contig(acc, s, rs, sv, bias, y)
    if acc.shape[0] < M or col0 < 0 or col0 + N > acc.shape[1]:
        raise ValueError(f'post: accumulator {tuple(acc.shape)} does not hold columns {col0}..{col0 + N} of {M} rows')
    if (sv is not None and sv.numel() != N) or (rs is not None and rs.numel() != N) or (bias is not None and bias.numel() != N):
        raise ValueError('post: sv / rs / bias must have N elements')
    call('tcq_post', ptr(acc), _dt(acc, (0, 1, 3), 'post acc'), acc.shape[1], col0, ptr(s), ptr(rs), ptr(sv), ptr(bias), ptr(y),
         _dt(y, (0, 1, 2), 'post y'), M, N, stream())


# ----------------------------------------------------------------------------------------------------------- MLP middles
def _ldq(q4):
    """ldq of a q4 output: the column count of a (K / 4, ldq) word tensor, LDQ_TOKEN_BLOCKS for a token-block tensor."""
    return 0 if q4 is None else LDQ_TOKEN_BLOCKS if q4.dim() == 4 else q4.shape[1]


def mid2(acc, s, rs, sv, su, q=None, q4=None, scale=None, gelu_lut=None):
    """Gated-MLP middle: acc (M, lda >= 2N) gate | up (int32 scaled by s, rs; FP32 already scaled; BF16 scaled by rs); rs, sv
    concatenated (2N); su = input signs of the down projection (N) -> q / q4, scale (reference kernels.py:640-643)."""
    M, N = acc.shape[0], su.numel()
    _contig(acc, s, rs, sv, su, q, q4, scale)
    lut = gelu_table(acc.device) if gelu_lut is None else gelu_lut
    call('tcq_mid2', ptr(acc), _dt(acc, (0, 1, 3), 'mid2 acc'), acc.shape[1], ptr(s), ptr(rs), ptr(sv), ptr(lut), ptr(su), ptr(q),
         ptr(q4), _ldq(q4), ptr(scale), M, N, stream())


def mid1(acc, s, rs, sv, bias, su, q=None, q4=None, scale=None, gelu_lut=None):
    """Plain-MLP middle: acc (M, N) of the first layer; su = input signs of the second layer (reference kernels.py:646-650)."""
    M, N = acc.shape[0], su.numel()
    _contig(acc, s, rs, sv, bias, su, q, q4, scale)
    lut = gelu_table(acc.device) if gelu_lut is None else gelu_lut
    call('tcq_mid1', ptr(acc), _dt(acc, (0, 1, 3), 'mid1 acc'), acc.shape[1], ptr(s), ptr(rs), ptr(sv), ptr(bias), ptr(lut),
         ptr(su), ptr(q), ptr(q4), _ldq(q4), ptr(scale), M, N, stream())


def pre2(g, u, su, q=None, q4=None, scale=None):
    """x = BF16(g * u) * su -> block Walsh -> per-token INT8; g, u (M, K) BF16 (reference kernels.py:631-633)."""
    M, K = g.shape
    if g.dtype != torch.bfloat16 or u.dtype != torch.bfloat16:
        raise TypeError('pre2: g and u must be bfloat16')
    _contig(g, u, su, q, q4, scale)
    call('tcq_pre2', ptr(g), ptr(u), ptr(su), ptr(q), ptr(q4), _ldq(q4), ptr(scale), M, K, stream())


# ------------------------------------------------------------------------------------------- norms around the projections
def _bf16(t, what):
    if t.dtype != torch.bfloat16:
        raise TypeError(f'{what} must be bfloat16')


def rmsnorm(x, w, eps, y):
    """Gemma RMSNorm, BF16 x (M, K) -> y, w (K,) BF16; FP32 arithmetic with a sum order fixed by K."""
    M, K = x.shape
    _bf16(x, 'rmsnorm x'), _bf16(w, 'rmsnorm w'), _bf16(y, 'rmsnorm y')
    _contig(x, w, y)
    call('tcq_rmsnorm', ptr(x), ptr(w), float(eps), ptr(y), M, K, stream())
    return y


def norm_pre(x, w, eps, su, q=None, q4=None, scale=None):
    """rmsnorm then pre(., su) in one launch: q / q4 / scale of fwht(RMSNorm(x) * su)."""
    M, K = x.shape
    _bf16(x, 'norm_pre x'), _bf16(w, 'norm_pre w')
    _contig(x, w, su, q, q4, scale)
    call('tcq_norm_pre', ptr(x), ptr(w), float(eps), ptr(su), ptr(q), ptr(q4), _ldq(q4), ptr(scale), M, K, stream())


def post_add_norm_pre(acc, s, rs, sv, bias, x, xout, w=None, eps=0.0, su=None, q=None, q4=None, scale=None, col0=0):
    """xout = bf16(x + post(acc ...)) and, with w, q / q4 / scale of fwht(RMSNorm(xout) * su), one launch. acc as post, or
    an int32 (P, M, lda) tensor of P = 2 / 4 K parts of one product (summed in int32 before scaling)."""
    M, N = x.shape
    _bf16(x, 'post_add_norm_pre x'), _bf16(xout, 'post_add_norm_pre xout')
    _contig(acc, s, rs, sv, bias, x, xout, w, su, q, q4, scale)
    adt = _dt(acc, (0, 1, 3), 'post_add_norm_pre acc')
    if acc.dim() == 3:
        if acc.dtype != torch.int32 or acc.shape[0] not in K_PARTS or acc.shape[1] != M:
            raise ValueError(f'post_add_norm_pre: K parts must be int32 (2 or 4, {M}, lda), got {tuple(acc.shape)} {acc.dtype}')
        adt |= K_PARTS[acc.shape[0]]
    elif acc.shape[0] < M:
        raise ValueError(f'post_add_norm_pre: accumulator {tuple(acc.shape)} has fewer than {M} rows')
    lda = acc.shape[-1]
    if col0 < 0 or col0 + N > lda:
        raise ValueError(f'post_add_norm_pre: columns {col0}..{col0 + N} exceed the accumulator width {lda}')
    call('tcq_post_add_norm_pre', ptr(acc), adt, lda, col0, ptr(s), ptr(rs), ptr(sv), ptr(bias), ptr(x), ptr(xout), ptr(w),
         float(eps), ptr(su), ptr(q), ptr(q4), _ldq(q4), ptr(scale), M, N, stream())
    return xout


# ------------------------------------------------------------------------------------------------------------- attention
def attend(q, k_cache, v_cache, k_new, v_new, heads, causal_offset=None, o=None, su=None, q8=None, scale=None, q4=None):
    """Multi-query attention (H <= 8 heads, head dim 256), BF16: keys / values = cache rows (or None) then the new rows.
    Writes o (M, H * 256) BF16 and / or, with su, q8 / q4 / scale of the rotate + quantize prologue of the next projection
    (q4 as in pre: word layout or token blocks)."""
    M = q.shape[0]
    P = 0 if k_cache is None else k_cache.shape[0]
    for t in (q, k_cache, v_cache, k_new, v_new, o):
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError('attend: BF16 tensors only')
    _contig(q, k_cache, v_cache, k_new, v_new, o, su, q8, q4, scale)
    D = k_new.shape[1]
    nc = int(_lib.lib().tcq_attend_chunks(P, M))
    part = torch.empty(M * nc * heads * (D + 4), dtype=torch.float32, device=q.device)
    call('tcq_attend_q4', ptr(q), ptr(k_cache), ptr(v_cache), P, ptr(k_new), ptr(v_new), M, heads, D,
         -1 if causal_offset is None else int(causal_offset), ptr(part), ptr(o), ptr(su), ptr(q8), ptr(q4), _ldq(q4), ptr(scale),
         stream())
    return o


def attend_parts(q, k_cache, v_cache, k_new, v_new, heads, causal_offset=None):
    """The first half of attend: the chunk partials of every token (tcq_attend_parts), without the merge. Returns
    (part, chunks, keys, causal) for prologue_attn."""
    M = q.shape[0]
    P = 0 if k_cache is None else k_cache.shape[0]
    for t in (q, k_cache, v_cache, k_new, v_new):
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError('attend_parts: BF16 tensors only')
    _contig(q, k_cache, v_cache, k_new, v_new)
    D = k_new.shape[1]
    nc = int(_lib.lib().tcq_attend_chunks(P, M))
    part = torch.empty(M * nc * heads * (D + 4), dtype=torch.float32, device=q.device)
    causal = -1 if causal_offset is None else int(causal_offset)
    call('tcq_attend_parts', ptr(q), ptr(k_cache), ptr(v_cache), P, ptr(k_new), ptr(v_new), M, heads, D, causal, ptr(part), stream())
    return part, nc, P + M, causal


def attend_post_parts(z, segments, k_cache, v_cache, k_out, v_out, heads, causal_offset=None):
    """The q / k / v epilogue of a one-token FP32 product row z (1, ldz) and attend_parts in one launch
    (tcq_attend_post_parts): segments = ((col0, sv) of q, of k, of v); the new key / value rows go to k_out / v_out
    ((1, 256) BF16, e.g. row P of a cache). Returns (part, chunks, keys, causal) for prologue_attn."""
    if z.dtype != torch.float32 or z.dim() != 2 or z.shape[0] != 1:
        raise TypeError('attend_post_parts: one FP32 row of z')
    for t in (k_cache, v_cache, k_out, v_out):
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError('attend_post_parts: BF16 cache and outputs')
    _contig(z, k_cache, v_cache, k_out, v_out, *(sv for _, sv in segments))
    P = 0 if k_cache is None else k_cache.shape[0]
    D = k_out.shape[-1]
    nc = int(_lib.lib().tcq_attend_chunks(P, 1))
    part = torch.empty(nc * heads * (D + 4), dtype=torch.float32, device=z.device)
    causal = -1 if causal_offset is None else int(causal_offset)
    zp = [z.data_ptr() + 4 * c0 for c0, _ in segments]
    call('tcq_attend_post_parts', *zp, *(ptr(sv) for _, sv in segments), ptr(k_cache), ptr(v_cache), P, ptr(k_out), ptr(v_out),
         heads, D, causal, ptr(part), stream())
    return part, nc, P + 1, causal


def prologue_attn(parts, heads, su, q=None, scale=None):
    """The attention prologue of a one-token product (tcq_prologue with part): the merge of attend_parts' partials of 8
    heads, then the rotate + quantize of the BF16 row with signs su; q / scale: optional copies of the INT8 row and its
    scale. Returns (descriptor, K)."""
    part, nc, keys, causal = parts
    if part.numel() != nc * heads * (256 + 4):
        raise ValueError('prologue_attn: the partials of one token')
    _contig(part, su, q, scale)
    st = _lib.Prologue(None, 3, 0, 0, None, None, None, None, None, None, None, 0.0, ptr(su), ptr(q), ptr(scale), ptr(part), nc, keys,
                       causal, heads)
    return st, heads * 256


def attend_static(q, k_cache, v_cache, k_new, v_new, heads, causal_offset=None, o=None, su=None, q8=None, scale=None, q4=None):
    """attend without a workspace allocation: the library's own per-device scratch array (tcq_attend_q4_static). For code
    that must not allocate (e.g. under graph capture); calls that overlap on one device race."""
    M = q.shape[0]
    P = 0 if k_cache is None else k_cache.shape[0]
    for t in (q, k_cache, v_cache, k_new, v_new, o):
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError('attend_static: BF16 tensors only')
    _contig(q, k_cache, v_cache, k_new, v_new, o, su, q8, q4, scale)
    call('tcq_attend_q4_static', ptr(q), ptr(k_cache), ptr(v_cache), P, ptr(k_new), ptr(v_new), M, heads, k_new.shape[1],
         -1 if causal_offset is None else int(causal_offset), ptr(o), ptr(su), ptr(q8), ptr(q4), _ldq(q4), ptr(scale), stream())
    return o


# -------------------------------------------------------------------------------------------------------------- products
def gemv_descriptors(layers):
    """[(wdev, tlut, row_scale, z), ...] -> device array of tcq_gemv_layer (4 pointers + rows_per_table each; z (M, m) gives
    m, a (G, 512, 2) tlut gives m / G rows per table). Keep the tensors alive."""
    flat = []
    for wdev, tlut, row_scale, z in layers:
        _contig(wdev, tlut, row_scale, z)
        G = _groups(tlut)
        flat += [ptr(wdev), ptr(tlut), ptr(row_scale), ptr(z), 0 if G == 1 else z.shape[-1] // G]
    dev = layers[0][0].device
    desc = torch.tensor(flat, dtype=torch.int64).to(dev)
    desc.rows_per_table = sorted(set(flat[4::5]))         # the launch plan needs one common value (checked by gemv_f16)
    return desc


def gemv_f16(desc, h16, hscale, m, n, rows_per_table=None):
    """Batched FP16-table decode-GEMV: for every layer in desc, z (M, m) = (h16 Q^T) * hscale * row_scale (M <= 16). The
    rows per table come from the descriptors (all layers must agree); a rows_per_table argument must equal them."""
    M = h16.shape[0]
    _contig(h16, hscale)
    rpt = getattr(desc, 'rows_per_table', None)
    if rpt is None:
        raise ValueError('gemv_f16: descriptors must come from gemv_descriptors')
    if len(rpt) != 1:
        raise ValueError(f'gemv_f16: the layers have different rows per table {rpt}')
    if rows_per_table is not None and rows_per_table != rpt[0]:
        raise ValueError(f'gemv_f16: rows_per_table {rows_per_table} differs from the descriptors ({rpt[0]})')
    call('tcq_gemv_f16_groups', ptr(desc), desc.numel() // 5, ptr(h16), ptr(hscale), M, m, n, rpt[0], stream())


def gemv_post_descriptors(layers):
    """[(wdev, tlut, row_scale, sv, bias, y), ...] -> device array of tcq_gemv_post_layer (single-table layers; bias may be
    None). Keep the tensors alive."""
    flat = []
    for wdev, tlut, row_scale, sv, bias, y in layers:
        _contig(wdev, tlut, row_scale, sv, bias, y)
        if _groups(tlut) != 1:
            raise ValueError('the fused output rotation takes single-table layers')
        flat += [ptr(wdev), ptr(tlut), ptr(row_scale), 0, ptr(sv), ptr(bias) or 0, ptr(y)]
    return torch.tensor(flat, dtype=torch.int64).to(layers[0][0].device)


def gemv_f16_post(desc, h16, hscale, m, n, y_dtype):
    """Layer stream with the output rotation fused: y = walsh((h16 Q^T) * hscale * row_scale) * sv (+ bias) per layer, one
    launch (bit-identical to gemv_f16 followed by post / postg)."""
    M = h16.shape[0]
    _contig(h16, hscale)
    call('tcq_gemv_f16_post', ptr(desc), desc.numel() // 7, ptr(h16), ptr(hscale), M, m, n, DTYPE[y_dtype], stream())


def layer_f16(x, su, wdev, tlut, row_scale, sv, bias, y, z, counter):
    """One launch of a whole FP16-table layer (tcq_layer_f16): y (M, m) = walsh(walsh(x * su) Q^T * row_scale) * sv (+ bias),
    bit-identical to pre_h16 -> gemv_f16 -> post. z (M, m) float32 and counter (one int32, zero before the first call, left
    zero) are its workspace."""
    M, n = x.shape
    m = row_scale.numel()
    _contig(x, su, wdev, tlut, row_scale, sv, bias, y, z, counter)
    if tuple(y.shape) != (M, m) or z.dtype != torch.float32 or z.numel() < M * m:
        raise ValueError(f'layer_f16: y must be ({M}, {m}) and z hold {M * m} float32')
    if su.numel() != n or sv.numel() != m or (bias is not None and bias.numel() != m) or _groups(tlut) != 1:
        raise ValueError('layer_f16: su (n,), sv (m,), bias (m,) and one (512, 2) table')
    if counter.dtype != torch.int32 or counter.numel() < 1:
        raise ValueError('layer_f16: counter must be an int32 tensor')
    call('tcq_layer_f16', ptr(x), _dt(x, (0, 1, 2), 'layer_f16 x'), ptr(su), ptr(wdev), ptr(tlut), ptr(row_scale), ptr(sv),
         ptr(bias), ptr(y), DTYPE[y.dtype], M, m, n, ptr(z), ptr(counter), stream())


def pre_gemv_f16(x, su, wdev, tlut, row_scale, z):
    """Input rotation and decode-GEMV of an FP16-table layer in one launch (tcq_pre_gemv_f16): z (M, m) float32 =
    walsh(x * su) Q^T * row_scale, bit-identical to pre_h16 -> gemv_f16; post(z, ...) completes the layer."""
    M, n = x.shape
    m = row_scale.numel()
    _contig(x, su, wdev, tlut, row_scale, z)
    if z.dtype != torch.float32 or tuple(z.shape) != (M, m):
        raise ValueError(f'pre_gemv_f16: z must be ({M}, {m}) float32')
    if su.numel() != n or _groups(tlut) != 1:
        raise ValueError('pre_gemv_f16: su (n,) and one (512, 2) table')
    call('tcq_pre_gemv_f16', ptr(x), _dt(x, (0, 1, 2), 'pre_gemv_f16 x'), ptr(su), ptr(wdev), ptr(tlut), ptr(row_scale), M, m, n,
         ptr(z), stream())


_SEG = None


def _seg_dtype():
    global _SEG
    if _SEG is None:
        import numpy as np
        _SEG = np.dtype([('acc', '<u8'), ('rs', '<u8'), ('sv', '<u8'), ('bias', '<u8'), ('y', '<u8'), ('lda', '<i4'),
                         ('col0', '<i4'), ('N', '<i4'), ('gelu', '<i4')])
        assert _SEG.itemsize == 56
    return _SEG


def post_segments(segs, device):
    """[(acc, col0, rs, sv, bias, y, gelu), ...] -> device array of tcq_post_seg. acc: (M, lda) tensor; y: (M, N) tensor.
    Keep the tensors alive while the array is in use (its pointers are baked in, as in a captured graph)."""
    import numpy as np
    a = np.zeros(len(segs), dtype=_seg_dtype())
    for i, (acc, col0, rs, sv, bias, y, gelu) in enumerate(segs):
        _contig(acc, rs, sv, bias, y)
        N = y.shape[1]
        if col0 < 0 or col0 + N > acc.shape[1] or sv.numel() != N or (rs is not None and rs.numel() != N):
            raise ValueError(f'segment {i}: columns {col0}..{col0 + N} do not fit the accumulator / scales')
        if rs is None and acc.dtype != torch.float32:
            raise ValueError(f'segment {i}: an {acc.dtype} accumulator needs its row scale')
        a[i] = (ptr(acc), ptr(rs) or 0, ptr(sv), ptr(bias) or 0, ptr(y), acc.shape[1], col0, N, int(bool(gelu)))
    return torch.from_numpy(a.view(np.uint8).copy()).to(device)


def post_batched(desc, nseg, acc_dtype, y_dtype, s, M, maxN, gelu_lut=None):
    """Batched epilogue over nseg segments of post_segments (a device descriptor array; the batched form of the reference's
    kernels.postg, kernels.py:618-628): one workgroup per (token, segment). acc_dtype / y_dtype: torch dtypes shared by all
    segments."""
    call('tcq_postg', ptr(desc), nseg, DTYPE[acc_dtype], ptr(s), ptr(gelu_lut), DTYPE[y_dtype], M, maxN, stream())


def _side_by_side(acc, s, rs, sv, bias, ys):
    """Checks of the reference's three-layer epilogue arguments: columns, rs / sv / bias concatenated, BF16 outputs."""
    M = ys[0].shape[0]
    n = [y.shape[1] for y in ys]
    _contig(acc, s, rs, sv, bias, *ys)
    if acc.shape[0] < M or acc.shape[1] < sum(n):
        raise ValueError(f'accumulator {tuple(acc.shape)} does not hold {M} rows of {sum(n)} columns')
    if sv.numel() != sum(n) or (rs is not None and rs.numel() != sum(n)) or (bias is not None and bias.numel() != sum(n)):
        raise ValueError('rs / sv / bias must be the concatenations over the layers')
    if any(y.dtype != torch.bfloat16 or y.shape[0] != M for y in ys):
        raise TypeError('outputs must be (M, n) bfloat16')
    if acc.dtype == torch.int32 and (s is None or rs is None):
        raise ValueError('an int32 accumulator needs s and rs')
    return M, n


def post3(acc, s, rs, sv, bias, ys):
    """q / k / v in one launch (reference kernels.post3, kernels.py:618-621): rs, sv, bias concatenated over the three
    layers; ys = three (M, N_i) BF16 outputs."""
    M, n = _side_by_side(acc, s, rs, sv, bias, ys)
    if len(ys) != 3:
        raise ValueError('post3 takes three outputs')
    call('tcq_post3', ptr(acc), _dt(acc, (0, 1, 3), 'post3 acc'), ptr(s), ptr(rs), ptr(sv), ptr(bias), ptr(ys[0]), ptr(ys[1]),
         ptr(ys[2]), M, n[0], n[1], n[2], acc.shape[1], stream())


def postg(acc, s, rs, sv, bias, ys, gelu0=False):
    """Two or three layers sharing the accumulator row, one workgroup per (token, layer); optional GELU on the first
    (reference kernels.postg, kernels.py:624-628)."""
    M, n = _side_by_side(acc, s, rs, sv, bias, ys)
    if len(ys) not in (2, 3):
        raise ValueError('postg takes two or three outputs')
    y2, n2 = (ys[2], n[2]) if len(ys) == 3 else (None, 0)
    call('tcq_postg3', ptr(acc), _dt(acc, (0, 1, 3), 'postg acc'), ptr(s), ptr(rs), ptr(sv), ptr(bias), ptr(gelu_table(acc.device)),
         ptr(ys[0]), ptr(ys[1]), ptr(y2), M, n[0], n[1], n2, acc.shape[1], int(bool(gelu0)), stream())


def post_group(segs, acc_dtype, y_dtype, s, M, gelu_lut=None):
    """Epilogue of one layer group, at most MAX_SEGS segments [(acc, col0, rs, sv, bias, y, gelu), ...] as in post_segments,
    passed by value in the launch (reference kernels.post3 / postg as Group.posts calls them, kernels.py:618-628): every call
    may name new outputs, also under graph capture."""
    n = len(segs)
    if not 0 < n <= _lib.MAX_SEGS:
        raise ValueError(f'post_group takes 1..{_lib.MAX_SEGS} segments, got {n}')
    arr = (_lib.PostSeg * n)()
    for i, (acc, col0, rs, sv, bias, y, gelu) in enumerate(segs):
        _contig(acc, rs, sv, bias, y)
        N = y.shape[1]
        if col0 < 0 or col0 + N > acc.shape[1] or sv.numel() != N or (rs is not None and rs.numel() != N):
            raise ValueError(f'segment {i}: columns {col0}..{col0 + N} do not fit the accumulator / scales')
        if rs is None and acc.dtype != torch.float32:
            raise ValueError(f'segment {i}: an {acc.dtype} accumulator needs its row scale')
        if y.dtype != y_dtype or acc.dtype != acc_dtype:
            raise TypeError(f'segment {i}: dtypes differ from the group\'s')
        arr[i] = _lib.PostSeg(ptr(acc), ptr(rs), ptr(sv), ptr(bias), ptr(y), acc.shape[1], col0, N, int(bool(gelu)))
    call('tcq_post_group', arr, n, DTYPE[acc_dtype], ptr(s), ptr(gelu_lut), DTYPE[y_dtype], M, stream())


_GELU = {}


def gelu_table(device):
    """BF16 GELU (tanh approximation) of every BF16 bit pattern, computed by PyTorch on `device` (reference
    kernels.gelu_table, kernels.py:563-569): the fused kernels look the activation up instead of re-implementing it."""
    key = str(device)
    if key not in _GELU:
        x = torch.arange(65536, dtype=torch.int32, device=device).to(torch.int16).view(torch.bfloat16)
        _GELU[key] = torch.nn.functional.gelu(x, approximate='tanh').contiguous()
    return _GELU[key]


# ------------------------------------------------------------------------------------------------- small-M INT8 products
DOT4 = 0x2000
# One-token products (M == 1) on v_dot4c_i32_i8 instead of the 16 x 16 x 64 INT8 MFMA (TCQ_DOT4 in include/tcq_api.h);
# the int32 sums are the same either way. The default is the faster of the two on MI355X.
ONE_TOKEN_DOT = False


def _dot_flag(M, dot):
    if dot is None:
        dot = ONE_TOKEN_DOT and M == 1
    if dot and M != 1:
        raise ValueError('dot-product products take one token')
    return DOT4 if dot else 0


class SmallProduct:
    """A prepared small-M product over 1..4 segments [(w, t8, rs, out), ...]: out is a view whose first element is the
    segment's first output column of an (M, ldo) buffer (FP32 / BF16 scaled, or int32 sums); rs (m,) FP32 gives m. The
    descriptor array is built once (keep the tensors alive); __call__(q, s) launches on the current stream.
    resident False: w = tcq_repack words + t8 (fused decode; the segment form of reference kernels.gemm_tcq,
    kernels.py:671-673); resident True: w = (m, K) int8 weights (segment form of reference kernels.gemm_w8, kernels.py:662-668)."""

    def __init__(self, segs, ldo, resident=False):
        if not 1 <= len(segs) <= _lib.MAX_SEGS:
            raise ValueError(f'1 to {_lib.MAX_SEGS} segments')
        self.name = 'tcq_gemm_w8' if resident else 'tcq_gemm_tcq'
        self.arr = (_lib.GemmSeg * len(segs))()
        self.keep = segs
        self.odt = None
        self.K = None
        for i, (w, t8, rs, out) in enumerate(segs):
            _contig(w, t8, rs)
            d = _dt(out, (0, 1, 3), f'{self.name} out')
            if self.odt is not None and d != self.odt:
                raise TypeError('all segments need one output dtype')
            self.odt = d
            G = 1 if t8 is None else _groups(t8)
            if resident:
                if w.dim() != 2 or w.shape[0] != rs.numel() or w.dtype != torch.int8:
                    raise ValueError(f'segment {i}: resident weights must be ({rs.numel()}, K) int8')
                k = w.shape[1]
                if self.K is not None and k != self.K:
                    raise ValueError('all segments need one K')
                self.K = k
            self.arr[i] = _lib.GemmSeg(ptr(w), ptr(t8), ptr(rs), ptr(out), rs.numel(), 0 if G == 1 else rs.numel() // G)
        self.outs = [(o, rs.numel()) for _, _, rs, o in segs]
        self.n, self.ldo = len(segs), ldo
        self.fn = getattr(_lib.lib(), self.name)

    def __call__(self, q, s, parts=1, dot=None):
        """q (M, K) row-major, or a token-block tensor (M = s.numel() tokens; s is then required). parts 2 / 4: int32 outputs
        only, K parts written at out + p * M * ldo (see K_PARTS). dot: one-token products on dot-product instructions
        (DOT4); None = ONE_TOKEN_DOT at M == 1."""
        if q.dim() == 4:
            if s is None:
                raise ValueError('token-block activations need s (their token count)')
            M, K, odt = s.numel(), q.shape[1] * 16, self.odt | Q_TOKEN_BLOCKS
        else:
            (M, K), odt = q.shape, self.odt
        odt |= _dot_flag(M, dot)
        if parts != 1:
            if parts not in K_PARTS or self.odt != 3:
                raise ValueError('K parts: 2 or 4, int32 outputs only')
            odt |= K_PARTS[parts]
        if self.K is not None and K != self.K:
            raise ValueError(f'activations have K = {K}, the weights {self.K}')
        if s is not None and s.numel() < M:
            raise ValueError('fewer token scales than tokens')
        for o, m in self.outs:
            if o.storage_offset() + ((parts - 1) * M + M - 1) * self.ldo + m > o.untyped_storage().nbytes() // o.element_size():
                raise ValueError(f'an output buffer does not hold {parts} x {M} rows of stride {self.ldo}')
        rc = self.fn(self.arr, self.n, ptr(q), ptr(s), M, K, odt, self.ldo, stream())
        if rc:
            raise _lib.TcqError(f'{self.name} failed: {_lib.STATUS.get(rc, f"HIP error {rc}")} (status {rc})')

    def run_pro(self, pro, parts=1):
        """The product of one token whose INT8 activations come from the prologue `pro` (prologue() / prologue_pre()), run by
        every workgroup of the same launch (tcq_gemm_tcq_pro / tcq_gemm_w8_pro): FP32 z after the layer prologue, int32
        sums (optionally in K parts) after the rotate + quantize one."""
        st, K = pro
        if self.K is not None and K != self.K:
            raise ValueError(f'the prologue row has {K} columns, the weights {self.K}')
        if parts != 1 and (parts not in K_PARTS or self.odt != 3):
            raise ValueError('K parts: 2 or 4, int32 outputs only')
        for o, m in self.outs:
            if o.storage_offset() + (parts - 1) * self.ldo + m > o.untyped_storage().nbytes() // o.element_size():
                raise ValueError(f'an output buffer does not hold {parts} rows of stride {self.ldo}')
        fn = getattr(_lib.lib(), self.name + '_pro')
        rc = fn(self.arr, self.n, ctypes.byref(st), K, self.odt | (K_PARTS[parts] if parts > 1 else 0), self.ldo, stream())
        if rc:
            raise _lib.TcqError(f'{self.name}_pro failed: {_lib.STATUS.get(rc, f"HIP error {rc}")} (status {rc})')


def prologue(acc, s, rs, sv, x, xout, w, eps, su, q=None, scale=None, col0=0):
    """The one-token decoder-layer prologue of a product (tcq_prologue in include/tcq_api.h): the arguments of
    post_add_norm_pre for M = 1 with the norm and no bias. acc: the previous product's int32 sums, (1, lda) or K parts
    (P, 1, lda); x, xout (1, K) BF16; q (1, K) int8 / scale (1,) FP32: optional copies of the INT8 row and its scale.
    Returns (descriptor, K); keep the tensors alive until the launch has been issued."""
    K = x.shape[1]
    if x.shape[0] != 1 or xout.shape != x.shape:
        raise ValueError('prologue: one token, x and xout (1, K)')
    _bf16(x, 'prologue x'), _bf16(xout, 'prologue xout'), _bf16(w, 'prologue w')
    _contig(acc, s, rs, sv, x, xout, w, su, q, scale)
    if acc.dtype != torch.int32:
        raise TypeError('prologue: int32 accumulators')
    adt = 3
    if acc.dim() == 3:
        if acc.shape[0] not in K_PARTS or acc.shape[1] != 1:
            raise ValueError(f'prologue: K parts must be (2 or 4, 1, lda), got {tuple(acc.shape)}')
        adt |= K_PARTS[acc.shape[0]]
    lda = acc.shape[-1]
    if col0 < 0 or col0 + K > lda:
        raise ValueError(f'prologue: columns {col0}..{col0 + K} exceed the accumulator width {lda}')
    st = _lib.Prologue(ptr(acc), adt, lda, col0, ptr(s), ptr(rs), ptr(sv), None, ptr(x), ptr(xout), ptr(w), float(eps), ptr(su),
                       ptr(q), ptr(scale))
    return st, K


def prologue_pre(x, su, q=None, scale=None):
    """The rotate + quantize prologue of a one-token product (tcq_prologue without acc): tcq_pre of the (1, K) BF16 row x
    with signs su; q (1, K) int8 / scale (1,) FP32: optional copies of the INT8 row and its scale. Returns (descriptor, K)."""
    if x.dim() != 2 or x.shape[0] != 1:
        raise ValueError('prologue_pre: one token, x (1, K)')
    _bf16(x, 'prologue_pre x')
    _contig(x, su, q, scale)
    st = _lib.Prologue(None, 3, 0, 0, None, None, None, None, ptr(x), None, None, 0.0, ptr(su), ptr(q), ptr(scale))
    return st, x.shape[1]


def gemm_tcq_segments(segs, q, s, ldo, parts=1, dot=None):
    """One-shot fused decode + product over segments (see SmallProduct)."""
    _contig(q, s)
    SmallProduct(segs, ldo)(q, s, parts, dot)


def gemm_w8_segments(segs, q, s, ldo, parts=1, dot=None):
    """One-shot INT8-resident product over segments (see SmallProduct)."""
    _contig(q, s)
    SmallProduct(segs, ldo, resident=True)(q, s, parts, dot)


Z_W128T = 0x1000


def gemm_tcq_w128t(segs, q, s, dot=None, pro=None):
    """Fused decode + product of up to 4 segments [(words, t8, rs, zt), ...] at M <= 16 tokens whose FP32 z leaves the
    kernel after the first seven block-Walsh stages of each segment, block-transposed: zt (M, 128, m / 128) float32
    (TCQ_Z_W128T in include/tcq_api.h). q: token blocks (M = s.numel()) or (M, K) rows; dot as SmallProduct. pro: one token
    whose activations come from the decoder-layer prologue (prologue(); q and s unused). No reference counterpart."""
    arr = (_lib.GemmSeg * len(segs))()
    M = 1 if pro is not None else s.numel()
    for i, (w, t8, rs, zt) in enumerate(segs):
        _contig(w, t8, rs, zt)
        m = rs.numel()
        if zt.dtype != torch.float32 or tuple(zt.shape) != (M, 128, m // 128):
            raise ValueError(f'segment {i}: zt must be ({M}, 128, {m // 128}) float32')
        arr[i] = _lib.GemmSeg(ptr(w), ptr(t8), ptr(rs), ptr(zt), m, 0 if _groups(t8) == 1 else m // _groups(t8))
    if pro is not None:
        st, K = pro
        call('tcq_gemm_tcq_pro', arr, len(segs), ctypes.byref(st), K, 0 | Z_W128T, 128, stream())
        return
    blocks = q.dim() == 4
    K = q.shape[1] * 16 if blocks else q.shape[1]
    _contig(q, s)
    call('tcq_gemm_tcq', arr, len(segs), ptr(q), ptr(s), M, K, 0 | Z_W128T | (Q_TOKEN_BLOCKS if blocks else 0) | _dot_flag(M, dot),
         128, stream())


def glu_split(zt, sv, gelu_lut, p):
    """The gated-MLP middle after gemm_tcq_w128t of gate | up: zt (2, M, 128, N / 128) float32, sv (2N,) int8 signs of
    gate | up -> p (M, N) BF16 = bf16(gelu(g) * u); kernels.pre(p, down_su, ...) then equals mid2 bit for bit. N = 16384."""
    M, N = p.shape
    _contig(zt, sv, gelu_lut, p)
    if tuple(zt.shape) != (2, M, 128, N // 128) or zt.dtype != torch.float32 or p.dtype != torch.bfloat16 or sv.numel() != 2 * N:
        raise ValueError('glu_split: shapes do not match')
    call('tcq_glu_split', ptr(zt), N, ptr(sv), ptr(gelu_lut), ptr(p), M, stream())
    return p


def gemm_w8(W, q4, s, rs, z):
    """W (N, K) int8 resident, q4 (K/4, M) int32, z (M, N) FP32 = (float(acc) * s) * rs (reference kernels.gemm_w8,
    kernels.py:662-668)."""
    N, K = W.shape
    M = z.shape[0]
    _contig(W, q4, s, rs, z)
    if q4.shape[0] != K // 4 or q4.shape[1] < M or z.shape[1] != N or rs.numel() != N or s.numel() < M:
        raise ValueError('gemm_w8: shapes do not match')
    call('tcq_gemm_w8_q4', ptr(W), ptr(q4), q4.shape[1], ptr(s), ptr(rs), ptr(z), M, N, K, stream())


def gemm_tcq(bits, t8, q4, s, rs, z, K, bounds=(1 << 30, 1 << 30)):
    """Fused decode + product over the packed words as stored: bits of up to three layers concatenated along the rows,
    t8 their (512, 2) tables concatenated, tile rows below bounds[0] / bounds[1] / beyond on table 0 / 1 / 2; q4 (K/4, M),
    z (M, N) FP32 (reference kernels.gemm_tcq, kernels.py:671-673)."""
    M, N = z.shape
    _contig(bits, t8, q4, s, rs, z)
    if bits.numel() != (N // 16) * (K // 16) * 32 or q4.shape[0] != K // 4 or q4.shape[1] < M or rs.numel() != N:
        raise ValueError('gemm_tcq: shapes do not match')
    if t8.numel() < 1024 * (1 + (N // 16 > bounds[0]) + (N // 16 > bounds[1])):
        raise ValueError('gemm_tcq: fewer tables than the bounds select')
    call('tcq_gemm_tcq_q4', ptr(bits), ptr(t8), ptr(q4), q4.shape[1], ptr(s), ptr(rs), ptr(z), M, N, K, int(bounds[0]),
         int(bounds[1]), stream())


def gemm_bf16(a, w, out, sa=None, sw=None):
    """acc = a w^T with FP32 accumulation, a (M, K) / w (N, K) BF16; out (M, ldo) FP32 or BF16 of (acc * sa) * sw (either
    scale may be None). The W2 float path's product (Group.run_float, deploy/tcq_kernels/modules.py:117-144)."""
    M, K = a.shape
    N = w.shape[0]
    if a.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError('gemm_bf16: a and w must be bfloat16')
    _contig(a, w, sa, sw)
    if w.shape[1] != K or out.shape[0] != M or out.stride(1) != 1:
        raise ValueError('gemm_bf16: shapes do not match')
    call('tcq_gemm_bf16', ptr(a), ptr(w), ptr(sa), ptr(sw), ptr(out), _dt(out, (0, 1), 'gemm_bf16 out'), out.stride(0), M, N, K,
         stream())
    return out


# ------------------------------------------------------------------------------------------------------- W2 float path
def pre_h(x, su, h=None, hT=None):
    """Rotated activations as BF16: h (M, K) row-major and / or hT (K, ldh) with token = column, bf16(fwht(x * su))
    (reference kernels.pre_h, kernels.py:677-680). x (M, K) float32 / bfloat16 / float16."""
    M, K = x.shape
    if h is None and hT is None:
        raise ValueError('pre_h: give h and / or hT')
    _contig(x, su, h, hT)
    if any(t is not None and t.dtype != torch.bfloat16 for t in (h, hT)):
        raise TypeError('pre_h: h / hT must be bfloat16')
    if h is not None and tuple(h.shape) != (M, K):
        raise ValueError(f'pre_h: h {tuple(h.shape)} != {(M, K)}')
    if hT is not None and (hT.shape[0] != K or hT.shape[1] < M):
        raise ValueError(f'pre_h: hT {tuple(hT.shape)} does not hold ({K}, >= {M})')
    call('tcq_pre_h', ptr(x), _dt(x, (0, 1, 2), 'pre_h x'), ptr(su), ptr(h), ptr(hT), 0 if hT is None else hT.shape[1], M, K,
         stream())


def mid2_available(N):
    """Whether mid2 takes a gated-MLP middle of width N (reference kernels.mid2_available, kernels.py:636-638)."""
    return bool(_lib.lib().tcq_mid2_available(int(N)))


def gemmf_segments(segs, h, ldo, resident=False):
    """W2 float product over 1..4 segments [(w, t8, rs, out), ...] side by side: h (M, K) BF16 rotated activations; out a
    view whose first element is the segment's first output column of an (M, ldo) buffer, FP32 (= acc * rs) or BF16
    (= bf16(acc), the prefill rounding). resident False: w = tcq_repack words + t8 (fused decode, the segment form of
    reference kernels.gemmf_tcq); True: w = (m, K) int8 weights (segment form of kernels.gemmf_w8, kernels.py:689-696)."""
    if not 1 <= len(segs) <= _lib.MAX_SEGS:
        raise ValueError(f'1 to {_lib.MAX_SEGS} segments')
    if h.dtype != torch.bfloat16 or h.dim() != 2:
        raise TypeError('gemmf: h must be (M, K) bfloat16')
    _contig(h)
    M, K = h.shape
    arr = (_lib.GemmSeg * len(segs))()
    odt = None
    for i, (w, t8, rs, out) in enumerate(segs):
        _contig(w, t8, rs)
        d = _dt(out, (0, 1), 'gemmf out')
        if odt is not None and d != odt:
            raise TypeError('all segments need one output dtype')
        odt = d
        m = rs.numel()
        if resident and (w.dtype != torch.int8 or tuple(w.shape) != (m, K)):
            raise ValueError(f'segment {i}: resident weights must be ({m}, {K}) int8')
        if out.storage_offset() + (M - 1) * ldo + m > out.untyped_storage().nbytes() // out.element_size():
            raise ValueError(f'segment {i}: the output buffer does not hold {M} rows of stride {ldo}')
        G = 1 if t8 is None else _groups(t8)
        arr[i] = _lib.GemmSeg(ptr(w), ptr(t8), ptr(rs), ptr(out), m, 0 if G == 1 else m // G)
    call('tcq_gemmf_w8' if resident else 'tcq_gemmf_tcq', arr, len(segs), ptr(h), M, K, odt, ldo, stream())


def gemmf_w8(W, hT, rs, z):
    """W (N, K) int8 resident, hT (K, >= M) BF16 (token = column), z (M, N) FP32 = acc * rs with FP32 sums (reference
    kernels.gemmf_w8, kernels.py:689-691)."""
    N, K = W.shape
    M = z.shape[0]
    _contig(W, hT, rs, z)
    if hT.dtype != torch.bfloat16 or hT.shape[0] != K or hT.shape[1] < M or z.shape[1] != N or rs.numel() != N:
        raise ValueError('gemmf_w8: shapes do not match')
    call('tcq_gemmf_w8_hT', ptr(W), ptr(hT), hT.shape[1], ptr(rs), ptr(z), M, N, K, stream())


def gemmf_tcq(bits, t8, hT, rs, z, K, bounds=(1 << 30, 1 << 30)):
    """Fused decode + float product over the packed words as stored (bits and tables of up to three layers, bounds as
    gemm_tcq); hT (K, >= M) BF16, z (M, N) FP32 = acc * rs (reference kernels.gemmf_tcq, kernels.py:694-696)."""
    M, N = z.shape
    _contig(bits, t8, hT, rs, z)
    if bits.numel() != (N // 16) * (K // 16) * 32 or hT.dtype != torch.bfloat16 or hT.shape[0] != K or hT.shape[1] < M \
            or rs.numel() != N:
        raise ValueError('gemmf_tcq: shapes do not match')
    if t8.numel() < 1024 * (1 + (N // 16 > bounds[0]) + (N // 16 > bounds[1])):
        raise ValueError('gemmf_tcq: fewer tables than the bounds select')
    call('tcq_gemmf_tcq_hT', ptr(bits), ptr(t8), ptr(hT), hT.shape[1], ptr(rs), ptr(z), M, N, K, int(bounds[0]), int(bounds[1]),
         stream())


# ----------------------------------------------------------------------------------------------------------- W8A8 GEMM
def gemm_i8(a, w, out, sa=None, sw=None):
    """acc = a w^T exact in int32; out (M, ldo) int32 (acc), FP32 ((acc * sa) * sw) or BF16 of that. a (M, K), w (N, K) int8.
    The prefill product of the reference (torch._int_mm in Group.product, deploy/tcq_kernels/modules.py:86)."""
    M, K = a.shape
    N = w.shape[0]
    _contig(a, w, sa, sw)
    if w.shape[1] != K or out.shape[0] != M or out.stride(1) != 1:
        raise ValueError('gemm_i8: shapes do not match')
    call('tcq_gemm_i8', ptr(a), ptr(w), ptr(sa), ptr(sw), ptr(out), _dt(out, (0, 1, 3), 'gemm_i8 out'), out.stride(0), M, N, K,
         stream())
    return out
