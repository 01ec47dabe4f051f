"""The allocation-free attention entry point (tcq_attend_q4_static, called through the C ABI) against tcq_attend_q4 with a
caller-allocated workspace: BF16 outputs, INT8 rows and scales of the fused output-projection prologue bit-exact, on two
calls in a row (the second smaller, so stale scratch contents of the first would show), and a size beyond the scratch
array refused before launching."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = 'cuda'
H, D = 8, 256


def _case(M, P, causal, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    t = dict(q=torch.randn(M, H * D, generator=g, device=DEV).bfloat16(),
             kc=torch.randn(max(P, 1), D, generator=g, device=DEV).bfloat16() if P else None,
             vc=torch.randn(max(P, 1), D, generator=g, device=DEV).bfloat16() if P else None,
             kn=torch.randn(M, D, generator=g, device=DEV).bfloat16(),
             vn=torch.randn(M, D, generator=g, device=DEV).bfloat16(),
             su=(torch.randint(0, 2, (H * D,), generator=g, device=DEV) * 2 - 1).to(torch.int8))
    t.update(M=M, P=P, causal=causal)
    return t


def _outputs(M):
    from yanlongvla_amd import kernels as K
    return dict(o=torch.full((M, H * D), float('nan'), device=DEV).bfloat16(), q8=torch.zeros(M, H * D, dtype=torch.int8, device=DEV),
                q4=K.token_blocks(M, H * D, DEV).zero_(), scale=torch.zeros(M, device=DEV))


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _call(lib, c, out, part=None):
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [_p(c['q']), _p(c['kc']), _p(c['vc']), c['P'], _p(c['kn']), _p(c['vn']), c['M'], H, D, c['causal']]
    tail = [_p(out['o']), _p(c['su']), _p(out['q8']), _p(out['q4']), -16, _p(out['scale']), st]
    if part is None:
        return lib.tcq_attend_q4_static(*args, *tail)
    return lib.tcq_attend_q4(*args, _p(part), *tail)


def test_static_scratch_matches_caller_workspace():
    from yanlongvla_amd import _lib
    lib = _lib.lib()
    cases = [_case(50, 800, -1, 1), _case(3, 100, 100, 2)]        # expert chunk shape, then a smaller causal call
    for c in cases:
        print(f'case M={c["M"]} P={c["P"]} causal={c["causal"]}', flush=True)
        nc = lib.tcq_attend_chunks(c['P'], c['M'])
        part = torch.empty(c['M'] * nc * H * (D + 4), dtype=torch.float32, device=DEV)
        a, b = _outputs(c['M']), _outputs(c['M'])
        assert _call(lib, c, a, part) == 0
        assert _call(lib, c, b) == 0
        torch.cuda.synchronize()
        for k in ('o', 'q8', 'q4', 'scale'):
            assert torch.equal(a[k].view(torch.uint8), b[k].view(torch.uint8)), k
        assert torch.isfinite(b['o'].float()).all()


def test_static_scratch_refuses_sizes_beyond_the_array():
    from yanlongvla_amd import _lib
    lib = _lib.lib()
    cap = lib.tcq_attend_static_floats()
    assert cap == 1 << 21
    c = _case(800, 0, 0, 3)                        # 800 causal rows: 800 * 13 chunks * 8 heads * 260 floats > the array
    assert 800 * lib.tcq_attend_chunks(0, 800) * H * (D + 4) > cap
    assert _call(lib, c, _outputs(800)) == -4


FRESH_PROCESS = r'''
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + '/tests')
from yanlongvla_amd import _lib
from test_zz_no_alloc import _case, _outputs, _call, H, D
lib = _lib.lib()
torch.cuda.init()
c = _case(50, 800, -1, 4)
nc = lib.tcq_attend_chunks(c['P'], c['M'])
part = torch.empty(c['M'] * nc * H * (D + 4), dtype=torch.float32, device='cuda')
ref, out = _outputs(c['M']), _outputs(c['M'])
assert _call(lib, c, ref, part) == 0
torch.cuda.synchronize()
print('step: capture with the first static call of the process', flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    rc = _call(lib, c, out)
assert rc == 0, rc
for replay in range(3):
    for k, v in _outputs(c['M']).items():
        out[k].copy_(v)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    for k in ('o', 'q8', 'q4', 'scale'):
        assert torch.equal(ref[k].view(torch.uint8), out[k].view(torch.uint8)), (replay, k)
print('step: allocation check', flush=True)
torch.cuda.synchronize()
a0, f0 = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
assert _call(lib, c, out) == 0
torch.cuda.synchronize()
a1, f1 = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
assert (a0, f0) == (a1, f1), ((a0, f0), (a1, f1))
print('FRESH_PROCESS_OK', flush=True)
'''


def test_static_scratch_first_call_under_graph_capture():
    """In a fresh process, the first call of tcq_attend_q4_static (the per-device scratch lookup included) is recorded in a
    HIP graph; three replays, each after eager writes over the outputs, equal the caller-workspace call bit for bit; and
    an eager call changes neither PyTorch's allocated bytes nor the device's free memory."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, '-c', FRESH_PROCESS, str(root)], capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and 'FRESH_PROCESS_OK' in r.stdout
