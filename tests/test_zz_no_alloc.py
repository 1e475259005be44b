"""The allocation-free decode entry point (aila_hip_gqa_decode_noalloc),
called through the C ABI, against the workspace entry point
(aila_hip_gqa_decode) and the CPU oracle, on two calls in a row -- the
second smaller, so it runs over the first call's leftover split records in
the shared static scratch.

Bar: bit-exact against the workspace entry point given the same split plan
(both hold enough records for the planned splits here), and max relative
error 1e-2 against the fp32 oracle (the attention output tolerance).
"""
import ctypes

import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg

pytestmark = pytest.mark.gpu
ATTN_TOL = 1e-2


def _t(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()


def _np(t):
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def _relerr(a, r):
    return float(np.max(np.abs(a - r)) / max(float(np.max(np.abs(r))), 1e-30))


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _call(seed, B, Hq, Hkv, D, max_seq, L, lens=None):
    import torch
    import aila_amd
    lib = aila_amd.lib()
    print(f"noalloc case seed={seed} B={B} Hq={Hq} Hkv={Hkv} D={D} max_seq={max_seq} L={L}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    dq, dk, dv = _t(q), _t(kc), _t(vc)
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda") if lens is not None else None
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out_na = torch.empty_like(dq)
    rc = lib.aila_hip_gqa_decode_noalloc(_p(dq), _p(dk), _p(dv), _p(out_na), B, Hq, Hkv, D, max_seq, L,
                                         _p(sl) if sl is not None else None, stream)
    assert rc == 0, lib.aila_hip_last_error()
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out_ws = torch.empty_like(dq)
    rc = lib.aila_hip_gqa_decode(_p(dq), _p(dk), _p(dv), _p(out_ws), _p(ws), ws.numel(), B, Hq, Hkv, D, max_seq,
                                 L, _p(sl) if sl is not None else None, stream)
    assert rc == 0, lib.aila_hip_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ws)
    got = dg.bf16_to_f32(_np(out_na))
    for b in range(B):
        lb = L if lens is None else min(lens[b], L)
        want = dg.bf16_to_f32(oracle.attention_decode_baseline(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv,
                                                               D, max_seq, lb))[0]
        assert _relerr(got[b], want) <= ATTN_TOL, (b, lb)


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: config-5 head shape, 4 sequences; second: smaller, other D
    # and group size, per-sequence lengths -- it reads the scratch the first
    # call left behind only where it wrote it itself.
    _call(0x0A11, 4, 16, 4, 256, 5120, 5000)
    _call(0x0A12, 2, 8, 2, 128, 800, 700, lens=[700, 333])


def test_noalloc_rejects_sizes_beyond_the_scratch():
    import aila_amd
    lib = aila_amd.lib()
    cap = lib.aila_hip_gqa_decode_noalloc_max_bytes()
    assert cap == 8 << 20
    p = ctypes.c_void_p(256)   # never dereferenced: the size check fails first
    B, Hq, D = 4096, 16, 256   # two records per head need 142 MB
    rc = lib.aila_hip_gqa_decode_noalloc(p, p, p, p, B, Hq, 4, D, 1024, 100, None, None)
    assert rc == -1
    assert b"scratch" in lib.aila_hip_last_error()


_CAPTURE_SCRIPT = r'''
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import aila_amd
from aila_amd import datagen as dg
lib = aila_amd.lib()
B, Hq, Hkv, D, max_seq, L = 2, 16, 4, 256, 4096, 4000
def t(x):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()
q = t(dg.normal_bf16(0x0A13, 0, (B, Hq, D)))
kc = t(dg.normal_bf16(0x0A13, 1, (B, Hkv, max_seq, D)))
vc = t(dg.normal_bf16(0x0A13, 2, (B, Hkv, max_seq, D)))
lens = torch.tensor([4000, 2500], dtype=torch.int32, device="cuda")
out_g = torch.empty_like(q)
p = lambda x: ctypes.c_void_p(x.data_ptr())
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.stream(s):
    with torch.cuda.graph(g, stream=s):
        # the first no-alloc call of this process: its scratch lookup happens here
        rc = lib.aila_hip_gqa_decode_noalloc(p(q), p(kc), p(vc), p(out_g), B, Hq, Hkv, D, max_seq, L, p(lens),
                                             ctypes.c_void_p(s.cuda_stream))
assert rc == 0, lib.aila_hip_last_error()
ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
ref = aila_amd.gqa_decode(q, kc, vc, L, workspace=ws, seq_lens=lens)
torch.cuda.synchronize()
for i in range(3):
    out_g.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_g, ref), f"replay {i} differs"
    lens[1] = 2500 - 100 * (i + 1)          # eager work between replays: a shorter sequence
    ref = aila_amd.gqa_decode(q, kc, vc, L, workspace=ws, seq_lens=lens)
    torch.cuda.synchronize()
print("CAPTURE_OK")
'''


def test_noalloc_first_call_inside_graph_capture():
    """The scratch address is looked up on a device's first no-alloc call;
    here that first call is made under HIP graph capture (a fresh process),
    and the captured launch replays bit-exact against the workspace entry
    point, with the sequence lengths changed between replays."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc first call under capture (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout, r.stdout + r.stderr
