"""GPU parity: GQA decode over a window of the cache with attention sinks
(aila_hip_gqa_decode_window; ops::attention_decode's
AILA_ATTN_DECODE_WINDOW / _WINDOW_START / _SINK, AttentionOps.cpp:533-551,
598-616) against the oracle (pinned in tests/test_oracle_window.py).

Rows the window drops are NaN-poisoned in the cache: reading any of them
would turn the output into NaN. Tolerance: bf16 outputs within max relative
error 1e-2 of the fp32 oracle.
"""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _t(x):
    import torch
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _np(t):
    return t.detach().view(__import__("torch").int16).cpu().numpy().view(np.uint16)


def _rel(a, r):
    a = dg.bf16_to_f32(a).astype(np.float64)
    r = dg.bf16_to_f32(r).astype(np.float64)
    return float(np.max(np.abs(a - r)) / max(float(np.max(np.abs(r))), 1e-30))


def _kept(L, window, start, sink):
    if start < 0:
        start = max(512, window)
    if window <= 0 or L <= start:
        return np.ones(L, bool)
    w = min(L, window)
    s = min(sink, L - w)
    keep = np.zeros(L, bool)
    keep[:s] = True
    keep[L - w:] = True
    return keep


@pytest.mark.parametrize("B,Hq,Hkv,D,max_seq,L,lens,window,start,sink,split", [
    (2, 16, 4, 256, 6144, 6000, None, 1024, -1, 4, True),      # Qwen3.5 attention shape, sink of 4
    (2, 16, 4, 256, 6144, 6000, None, 1024, -1, 4, False),     # single pass
    (3, 8, 2, 128, 4096, 4000, [4000, 1800, 700], 512, 1024, 37, True),   # device lengths, one below start
    (1, 16, 8, 128, 2048, 2000, None, 100, 512, 0, True),      # tail only, ragged window
    (2, 8, 8, 64, 2048, 1999, [1999, 1500], 300, 512, 1300, True),  # sink and tail meet for one sequence
    (1, 16, 4, 256, 131136, 131072, None, 4096, -1, 4, True),  # a 4k window at the end of a 128k context
])
def test_decode_window(B, Hq, Hkv, D, max_seq, L, lens, window, start, sink, split):
    import torch
    import aila_amd
    seed = 3000 + D + window
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    lens_ = lens if lens is not None else [L] * B
    kc_d, vc_d = kc.copy(), vc.copy()
    for b in range(B):
        drop = ~_kept(lens_[b], window, start, sink)
        kc_d[b, :, :lens_[b]][:, drop] = 0x7FC0
        vc_d[b, :, :lens_[b]][:, drop] = 0x7FC0
        kc_d[b, :, lens_[b]:] = 0x7FC0
        vc_d[b, :, lens_[b]:] = 0x7FC0
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda") if split else None
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda") if lens is not None else None
    out = aila_amd.gqa_decode(_t(q), _t(kc_d), _t(vc_d), L, workspace=ws, seq_lens=sl, window=(window, start, sink))
    torch.cuda.synchronize()
    got = _np(out)
    want = oracle.attention_decode_window(q, kc, vc, B, Hq, Hkv, D, max_seq, L, window, start, sink,
                                          lens=np.array(lens_, np.int32))
    assert np.isfinite(dg.bf16_to_f32(got)).all(), "a dropped row was read"
    for b in range(B):
        assert _rel(got[b], want[b]) <= TOL, f"sequence {b}"


def test_window_off_is_the_plain_decode():
    import torch
    import aila_amd
    B, Hq, Hkv, D, max_seq, L = 2, 16, 4, 256, 4096, 3000
    q = dg.normal_bf16(3100, 0, (B, Hq, D))
    kc = dg.normal_bf16(3100, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(3100, 2, (B, Hkv, max_seq, D))
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    a = aila_amd.gqa_decode(_t(q), _t(kc), _t(vc), L, workspace=ws, window=(0, -1, 16))
    b = aila_amd.gqa_decode(_t(q), _t(kc), _t(vc), L, workspace=ws)
    torch.cuda.synchronize()
    assert np.array_equal(_np(a), _np(b))
