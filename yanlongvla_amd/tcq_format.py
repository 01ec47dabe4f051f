"""The packed TCQ deployment format on the device: one quantized Linear per `Layer`, files in `packed.safetensors`.

Mirrors deploy/tcq_kernels/tcq_format.py (Layer 80-107, load 230-237, the file schema 1-13) with the derived tensors made by
the HIP library instead of PyTorch ops:

packed.safetensors: per quantized Linear `name`
  <name>::bits       int16 view of the uint16 words (m/16 * n/16, 32): 512 bits per 16 x 16 tile
  <name>::tlut       FP16 (512, 2) table, or (G, 512, 2) row-group tables (rows split evenly into G contiguous groups, the
                     GR00T variants of baselines/groot/simpler/main_row/scripts/groot_tcq.py:154-175)
  <name>::row_scale  FP16 (m,)
  <name>::su, ::sv   int8 (n,), (m,) input / output signs of the two-sided block-Walsh rotation; a layer without ::sv is
                     one-sided (no output rotation: the GR00T "tcq" base, groot_tcq.py:187-191)
  <name>::col_scale  FP16 (n,), optional: column scales of the GR00T row-group records (groot_tcq.py:178-184), applied to
                     the rotated activations before they are quantized
Derived at load (tcq_snap on the device): t8 = clamp(round(tlut * g)), g = float(1 / max|tlut|) * 127; rs = row_scale / g.
Derived on demand: the repacked words of the fused products (tcq_repack), the INT8 weight (tcq_decode_i8).
"""
import os
from pathlib import Path

import torch

from . import kernels as K

ROOT = Path(os.environ.get('VLA_ROOT', '/projects/yanlongvla'))        # project root holding models/pi05_tcq/<row>/
ROW = 'tcq_raqft_d1'
TENSORS = ('bits', 'tlut', 'row_scale', 'su', 'sv')
OPTIONAL = ('sv', 'col_scale')


def block_widths(width):
    """Descending power-of-two Walsh blocks of a width (tcq_format.py:26-30): 4304 -> [4096, 128, 64, 16]."""
    out = []
    while width:
        b = 1 << (width.bit_length() - 1)
        out.append(b)
        width -= b
    return out


class Layer:
    """One quantized Linear on a device: the packed tensors, the INT8 table / FP32 row scale derived at load, and the
    device word layout of the fused products (made on first use). Same constructor as tcq_format.Layer (tcq_format.py:80-92)."""

    def __init__(self, name, tensors, bias=None, device='cuda'):
        self.name = name
        self.bits = tensors['bits'].to(device).view(torch.int16).contiguous()
        self.tlut = tensors['tlut'].to(device).to(torch.float16).contiguous()
        self.row_scale = tensors['row_scale'].to(device).to(torch.float16).contiguous()
        self.su = tensors['su'].to(device).to(torch.int8).contiguous()
        sv, cs = tensors.get('sv'), tensors.get('col_scale')
        self.sv = None if sv is None else sv.to(device).to(torch.int8).contiguous()
        self.col_scale = None if cs is None else cs.to(device).to(torch.float16).contiguous()
        self.m, self.n = self.row_scale.numel(), self.su.numel()
        if (self.sv is not None and self.sv.numel() != self.m) or (self.col_scale is not None and self.col_scale.numel() != self.n):
            raise ValueError(f'{name}: sv / col_scale do not fit a ({self.m}, {self.n}) layer')
        if not (self.bits.shape == ((self.m // 16) * (self.n // 16), 32) and self.m % 16 == 0 and self.n % 16 == 0):
            raise ValueError(f'{name}: bits {tuple(self.bits.shape)} do not fit a ({self.m}, {self.n}) layer of 16 x 16 tiles')
        if self.tlut.dim() == 3:                      # row-group tables (G, 512, 2): rows split evenly into G groups
            G = self.tlut.shape[0]
            if self.tlut.shape[1:] != (512, 2) or self.m % G or (self.m // G) % 16:
                raise ValueError(f'{name}: {G} row-group tables need (G, 512, 2) and m / G a multiple of 16 (m = {self.m})')
        elif self.tlut.shape != (512, 2):
            raise ValueError(f'{name}: table shape {tuple(self.tlut.shape)} != (512, 2)')
        self.groups = 1 if self.tlut.dim() == 2 else self.tlut.shape[0]
        self.t8, self.rs, self.gain = K.snap(self.tlut, self.row_scale)
        self.bias = None if bias is None else bias.float().to(device).contiguous()
        self._words = None
        self.bits_resident = True

    def words(self):
        """The tcq_repack layout of the words (cached)."""
        if self._words is None:
            if self.bits is None:
                raise RuntimeError(f'{self.name}: the bitstream was released at load (resident operating point)')
            self._words = K.repack(self.bits, self.m, self.n)
        return self._words

    def w8_reference(self, out=None):
        """INT8 weight (m, n) in the rotated basis: sign * t8[hash(state)] (tcq_format.py:97-98), decoded on the device."""
        out = torch.empty(self.m, self.n, dtype=torch.int8, device=self.bits.device) if out is None else out
        K.decode(self.bits, self.t8, out)
        return out

    def decode_f16(self, out=None):
        """FP16-table weight (m, n) in the rotated basis, before the row scale: sign * tlut[hash(state)]."""
        out = torch.empty(self.m, self.n, dtype=torch.float16, device=self.bits.device) if out is None else out
        K.decode_f16(self.bits, self.tlut, out)
        return out

    @property
    def one_sided(self):
        return self.sv is None

    def dense(self, table='fp16'):
        """Original-basis FP32 weight S_v H_m diag(r) Q diag(c) H_n S_u (tcq_format.py:100-107; the column scale and the
        one-sided form of groot_tcq.py:178-191), rotations by tcq_rht."""
        if table == 'fp16':
            q = self.decode_f16().float() * self.row_scale.float()[:, None]
        else:
            q = self.w8_reference().float() * self.rs[:, None]
        if self.col_scale is not None:
            q = q * self.col_scale.float()[None, :]
        w = torch.empty_like(q)
        K.rht(q, None, w)
        w = w * self.su.float()[None, :]
        if self.sv is None:
            return w
        w = w.t().contiguous()
        wt = torch.empty_like(w)
        K.rht(w, None, wt)
        return (wt * self.sv.float()[None, :]).t().contiguous()


def packed_path(row=ROW):
    """A row name -> ROOT/models/pi05_tcq/<row>/packed.safetensors (tcq_format.py:191-192); a path is taken as is."""
    p = Path(row)
    if p.suffix == '.safetensors' or p.exists():
        return p
    return ROOT / f'models/pi05_tcq/{row}/packed.safetensors'


def layer_names(row=ROW):
    """Names of the layers stored in a packed file (one per ::bits entry)."""
    from safetensors import safe_open
    with safe_open(str(packed_path(row)), framework='pt', device='cpu') as f:
        return [k[:-len('::bits')] for k in f.keys() if k.endswith('::bits')]


def load(row=ROW, device='cuda', names=None, biases=None):
    """{name: Layer} from a packed file (tcq_format.py:230-237)."""
    from safetensors import safe_open
    out = {}
    with safe_open(str(packed_path(row)), framework='pt', device='cpu') as f:
        keys = set(f.keys())
        for name in (names or [k[:-len('::bits')] for k in keys if k.endswith('::bits')]):
            t = {k: f.get_tensor(f'{name}::{k}') for k in TENSORS + ('col_scale',) if f'{name}::{k}' in keys}
            missing = [k for k in TENSORS if k not in t and k not in OPTIONAL]
            if missing:
                raise KeyError(f'{name}: packed file lacks {missing}')
            out[name] = Layer(name, t, bias=(biases or {}).get(name), device=device)
    return out


def save(tensors, path):
    """Write {name: {bits, tlut, row_scale, su[, sv][, col_scale]}} (CPU or device tensors) as a packed file."""
    from safetensors.torch import save_file
    flat = {}
    for name, t in tensors.items():
        for k in TENSORS + ('col_scale',):
            if t.get(k) is None:
                if k not in OPTIONAL:
                    raise KeyError(f'{name}: {k} is required')
                continue
            v = t[k].detach().cpu().clone()                  # members of a group may share one sign tensor
            flat[f'{name}::{k}'] = (v.view(torch.int16) if k == 'bits' else v).contiguous()
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    save_file(flat, str(path))
    return path


# ------------------------------------------------------------------------------------------- QTIP-official output
def from_qtip(rec):
    """One layer of QTIP-official output (baselines/quantize_qtip.py:66-84: trellis_int16, tlut_fp16, su_fp16, sv_fp16,
    wscale_fp32) -> the packed tensors {bits, tlut, row_scale, su, sv} (CPU tensors).

    QTIP's incoherence transform Wr = H_m S_V W S_U H_n (utils.matmul_hadUt on both sides, quantize_qtip.py:61) inverts to
    W = S_V H_m (Wscale Q) H_n S_U, the deploy format's S_v H_m diag(r) Q H_n S_u with the scalar Wscale as a constant row
    scale, whenever both Hadamards are the Sylvester ones the block Walsh uses: power-of-two m and n. The scale becomes FP16
    (the format's row-scale type). Layers padded for QTIP's other Hadamard sizes (4304 -> 4480, quantize_qtip.py:31) are
    refused: their transform is not a block Walsh."""
    su, sv = rec['su_fp16'].float(), rec['sv_fp16'].float()
    m, n = sv.numel(), su.numel()
    if m & (m - 1) or n & (n - 1):
        raise ValueError(f'QTIP layer {m} x {n}: only power-of-two dims use the Sylvester Hadamard of the block Walsh')
    bits = rec['trellis_int16'].contiguous().view(torch.int16).reshape(-1, 32)
    if bits.shape[0] != (m // 16) * (n // 16):
        raise ValueError(f'trellis holds {bits.shape[0]} tiles, a {m} x {n} layer has {(m // 16) * (n // 16)}')
    if not (torch.all(su.abs() == 1) and torch.all(sv.abs() == 1)):
        raise ValueError('sign vectors must hold +-1')
    wscale = rec['wscale_fp32'].reshape(-1)[0].float()
    return dict(bits=bits, tlut=rec['tlut_fp16'].to(torch.float16).reshape(512, 2).contiguous(),
                row_scale=wscale.to(torch.float16).expand(m).contiguous(), su=su.to(torch.int8), sv=sv.to(torch.int8))


def convert_qtip(files, path):
    """{layer name: QTIP-official per-layer .safetensors} -> one packed file at path."""
    from safetensors.torch import load_file
    return save({name: from_qtip(load_file(str(f))) for name, f in files.items()}, path)


# ------------------------------------------------------------------------------------------- GR00T fit records
def from_groot(rec):
    """One GR00T TCQ fit record -> the packed tensors {bits, tlut, row_scale, su[, sv][, col_scale]} (CPU tensors).

    The records (baselines/groot/simpler/main_row/scripts/groot_tcq.py:341-343 for the one- and two-sided bases, 470 for the
    row-group variants) hold `trellis` (QTIP pack_trellis of the 16 x 16 tiles in row-major tile order, state 8 r + p = row
    r, pair p of a tile: groot_tcq.pack / unpack, 218-228), `tlut` (512, 2) or (G, 512, 2) FP16, `row_scale` (m,) FP16,
    `signs` (n,) and optionally `signs_out` (m,) int8 and `col_scale` (n,) FP16, with the decoded weight
    W = [S_out H_m] diag(r) Q diag(c) H_n S_in (groot_tcq.decode / inverse_rotation, 178-191; inverse_rht = block Walsh then
    signs, groot_ptq.py:155-159). That is the deploy format's layer with bits = the trellis words (the same pack and tile
    order the reference's own packer copies unchanged for the pi0.5 records, deploy/tcq_kernels/tcq_format.py:204-207),
    su = signs, sv = signs_out (absent: one-sided) and the column scale kept. `rec` is the record or its `tensors` dict."""
    t = rec.get('tensors', rec)
    info = rec.get('tcq') if isinstance(rec.get('tcq'), dict) else None
    if info is not None and (info.get('L'), info.get('K'), info.get('V'), info.get('td')) not in ((16, 2, 2, 16), (None, None, None, None)):
        raise ValueError(f"record format {info}: the deploy path takes L = 16, K = 2, V = 2, 16 x 16 tiles")
    su = t['signs'].to(torch.int8).reshape(-1)
    rsc = t['row_scale'].to(torch.float16).reshape(-1)
    m, n = rsc.numel(), su.numel()
    bits = t['trellis'].contiguous().view(torch.int16).reshape(-1, 32)
    if bits.shape[0] != (m // 16) * (n // 16) or m % 16 or n % 16:
        raise ValueError(f'trellis holds {bits.shape[0]} tiles, a {m} x {n} layer has {(m // 16) * (n // 16)}')
    out = dict(bits=bits, tlut=t['tlut'].to(torch.float16).contiguous(), row_scale=rsc.contiguous(), su=su.contiguous())
    if t.get('signs_out') is not None:
        out['sv'] = t['signs_out'].to(torch.int8).reshape(-1).contiguous()
    if t.get('col_scale') is not None:
        out['col_scale'] = t['col_scale'].to(torch.float16).reshape(-1).contiguous()
    for k in ('su', 'sv'):
        if k in out and not torch.all(out[k].abs() == 1):
            raise ValueError(f'{k} must hold +-1')
    return out


def _read_record(path):
    """A record file: torch.save'd dicts of tensors (read without unpickling code) or safetensors."""
    path = Path(path)
    if path.suffix == '.safetensors':
        from safetensors.torch import load_file
        return load_file(str(path))
    return torch.load(str(path), map_location='cpu', weights_only=True)


def load_groot(files, device='cuda', biases=None):
    """{layer name: GR00T fit record file} -> {name: Layer}."""
    return {name: Layer(name, from_groot(_read_record(f)), bias=(biases or {}).get(name), device=device)
            for name, f in files.items()}


def convert_groot(files, path):
    """{layer name: GR00T fit record file} -> one packed file at path (sv / col_scale entries where the records hold them)."""
    return save({name: from_groot(_read_record(f)) for name, f in files.items()}, path)
