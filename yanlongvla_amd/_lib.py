"""ctypes binding of libtcq.so (the C ABI declared in include/tcq_api.h).

Mirrors the reference's kernel runtime (deploy/tcq_kernels/cuda_rt.py:79-108): tensors travel as raw device pointers,
ints as c_int, None as NULL, and every call is issued on torch.cuda.current_stream() so HIP graph captures record it. There is
no fallback: if the library is missing or was built for another architecture, loading fails loudly.
"""
import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / 'libtcq.so'

F32, BF16, F16, I32, I8 = 0, 1, 2, 3, 4
DTYPE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: I32, torch.int8: I8}
STATUS = {-1: 'invalid argument', -2: 'shape violates the format', -3: 'unsupported dtype', -4: 'unsupported size',
          -5: 'pointer not 16-byte aligned'}

_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
# name -> argument types (restype int unless listed in _RESTYPE)
SIGNATURES = {
    'tcq_version': [],
    'tcq_max_width': [],
    'tcq_snap': [_P, _P, _I, _P, _P, _P, _P],
    'tcq_repack': [_P, _P, _I, _I, _P],
    'tcq_repack_words': [_I, _I],
    'tcq_decode_i8': [_P, _P, _P, _I, _I, _P],
    'tcq_decode_i8_words': [_P, _P, _P, _I, _I, _P],
    'tcq_decode_f16': [_P, _P, _P, _I, _I, _P],
    'tcq_rht': [_P, _I, _I, _P, _P, _I, _I, _I, _I, _P],
    'tcq_pre': [_P, _I, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_pre_h16': [_P, _I, _P, _P, _P, _I, _I, _P],
    'tcq_quantize_rows': [_P, _I, _I, _P, _P, _I, _I, _P],
    'tcq_post': [_P, _I, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    'tcq_rmsnorm': [_P, _P, _F, _P, _I, _I, _P],
    'tcq_norm_pre': [_P, _P, _F, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_post_add_norm_pre': [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_attend_chunks': [_I, _I],
    'tcq_snap_groups': [_P, _I, _P, _I, _P, _P, _P, _P],
    'tcq_decode_i8_groups': [_P, _P, _I, _P, _I, _I, _P],
    'tcq_decode_f16_groups': [_P, _P, _I, _P, _I, _I, _P],
    'tcq_gemv_f16_groups': [_P, _I, _P, _P, _I, _I, _I, _I, _P],
    'tcq_gemv_f16_post': [_P, _I, _P, _P, _I, _I, _I, _I, _P],
    'tcq_layer_f16': [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P],
    'tcq_pre_gemv_f16': [_P, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P],
    'tcq_gemm_bf16': [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    'tcq_attend': [_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P],
    'tcq_attend_q4': [_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P, _P],
    'tcq_post_group': [_P, _I, _I, _P, _P, _I, _I, _P],
    'tcq_mid2': [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_mid1': [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_pre2': [_P, _P, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_postg': [_P, _I, _I, _P, _P, _I, _I, _I, _P],
    'tcq_gemv_f16': [_P, _I, _P, _P, _I, _I, _I, _P],
    'tcq_gemm_tcq': [_P, _I, _P, _P, _I, _I, _I, _I, _P],
    'tcq_gemm_w8': [_P, _I, _P, _P, _I, _I, _I, _I, _P],
    'tcq_gemm_i8': [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    'tcq_post3': [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    'tcq_postg3': [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    'tcq_gemm_w8_q4': [_P, _P, _I, _P, _P, _P, _I, _I, _I, _P],
    'tcq_gemm_tcq_q4': [_P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    'tcq_attend_q4_static': [_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _P],
    'tcq_attend_static_floats': [],
    'tcq_pre_cs': [_P, _I, _P, _P, _P, _P, _I, _P, _I, _I, _P],
    'tcq_pre_h': [_P, _I, _P, _P, _P, _I, _I, _I, _P],
    'tcq_mid2_available': [_I],
    'tcq_gemmf_tcq': [_P, _I, _P, _I, _I, _I, _I, _P],
    'tcq_gemmf_w8': [_P, _I, _P, _I, _I, _I, _I, _P],
    'tcq_gemmf_w8_hT': [_P, _P, _I, _P, _P, _I, _I, _I, _P],
    'tcq_gemmf_tcq_hT': [_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P],
    'tcq_glu_split': [_P, _I, _P, _P, _P, _I, _P],
    'tcq_gemm_tcq_pro': [_P, _I, _P, _I, _I, _I, _P],
    'tcq_gemm_w8_pro': [_P, _I, _P, _I, _I, _I, _P],
    'tcq_attend_parts': [_P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P],
    'tcq_attend_post_parts': [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _P, _P],
}
_RESTYPE = {'tcq_version': ctypes.c_char_p, 'tcq_repack_words': _L, 'tcq_attend_static_floats': ctypes.c_size_t}

MAX_SEGS = 4


class PostSeg(ctypes.Structure):
    """tcq_post_seg (include/tcq_api.h)."""
    _fields_ = [('acc', ctypes.c_void_p), ('rs', ctypes.c_void_p), ('sv', ctypes.c_void_p), ('bias', ctypes.c_void_p),
                ('y', ctypes.c_void_p), ('lda', ctypes.c_int), ('col0', ctypes.c_int), ('N', ctypes.c_int),
                ('gelu', ctypes.c_int)]


class GemmSeg(ctypes.Structure):
    """tcq_gemm_seg (include/tcq_api.h)."""
    _fields_ = [('w', ctypes.c_void_p), ('t8', ctypes.c_void_p), ('rs', ctypes.c_void_p), ('out', ctypes.c_void_p),
                ('m', ctypes.c_int), ('rows_per_table', ctypes.c_int)]


class Prologue(ctypes.Structure):
    """tcq_prologue (include/tcq_api.h)."""
    _fields_ = [('acc', ctypes.c_void_p), ('acc_dtype', ctypes.c_int), ('lda', ctypes.c_int), ('col0', ctypes.c_int),
                ('s', ctypes.c_void_p), ('rs', ctypes.c_void_p), ('sv', ctypes.c_void_p), ('bias', ctypes.c_void_p),
                ('x', ctypes.c_void_p), ('xout', ctypes.c_void_p), ('w', ctypes.c_void_p), ('eps', ctypes.c_float),
                ('su', ctypes.c_void_p), ('q', ctypes.c_void_p), ('scale', ctypes.c_void_p), ('part', ctypes.c_void_p),
                ('chunks', ctypes.c_int), ('keys', ctypes.c_int), ('causal', ctypes.c_int), ('heads', ctypes.c_int)]


_state = {}
_lock = threading.Lock()


class TcqError(RuntimeError):
    pass


def lib():
    """The loaded library (loaded once). Raises if libtcq.so has not been built."""
    if 'lib' not in _state:
        with _lock:
            if 'lib' not in _state:
                if not LIB_PATH.exists():
                    raise TcqError(f'{LIB_PATH} is missing: build it with `python -m yanlongvla_amd.build` '
                                   '(there is no CPU fallback)')
                L = ctypes.CDLL(str(LIB_PATH))
                for name, args in SIGNATURES.items():
                    f = getattr(L, name)
                    f.argtypes = args
                    f.restype = _RESTYPE.get(name, ctypes.c_int)
                _state['lib'] = L
    return _state['lib']


def ptr(t):
    """Device pointer of a tensor (None -> NULL). Refuses CPU tensors: the library only takes device memory."""
    if t is None:
        return None
    if not t.is_cuda:
        raise TcqError('libtcq takes device tensors only (got a CPU tensor)')
    return t.data_ptr()


def stream():
    return torch.cuda.current_stream().cuda_stream


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        what = STATUS.get(rc, f'HIP error {rc}')
        raise TcqError(f'{name} failed: {what} (status {rc})')
    return rc


def version():
    return lib().tcq_version().decode()
