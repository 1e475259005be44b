"""Seeded sweeps of GPU parity over shapes and lengths the targeted tests do
not pin one by one: split-K decode with device-side lengths (each sequence's
rows shared evenly by the launched splits) and prefill over a cached prefix
with and without the key split. Each case is checked against the CPU oracle
(AttentionOps.cpp:73-166 for decode, :2308-2507 for the cached prefill)
within the attention tolerance, with NaN in every cache row past the
attended range."""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg

pytestmark = pytest.mark.gpu
ATTN_TOL = 1e-2


def _t(x):
    import torch
    if x.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _np(t):
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def _relerr(a, r):
    return float(np.max(np.abs(a - r)) / max(float(np.max(np.abs(r))), 1e-30))


def _decode_cases():
    rng = np.random.default_rng(0x5EE9)
    cases = []
    for i in range(8):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 4, 8]))
        Hkv = int(rng.choice([1, 2, 4]))
        B = int(rng.integers(1, 6))
        bound = int(rng.integers(64, 3000))
        lens = [int(x) for x in rng.integers(1, bound + 1, size=B)]
        lens[0] = min(lens[0], int(rng.choice([1, 15, 16, 17])))   # short sequences beside long ones
        cases.append((i, D, G, Hkv, B, bound, lens))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,B,bound,lens", _decode_cases())
def test_sweep_decode_device_lengths(i, D, G, Hkv, B, bound, lens):
    import torch
    import aila_amd
    Hq = Hkv * G
    max_seq = bound + 7
    seed = 0x5EE0 + i
    print(f"sweep decode {i}: D={D} G={G} Hkv={Hkv} B={B} bound={bound} lens={lens}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    for b, L in enumerate(lens):
        kc[b, :, L:] = 0x7FC0
        vc[b, :, L:] = 0x7FC0
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = aila_amd.gqa_decode(_t(q), _t(kc), _t(vc), bound, workspace=ws, seq_lens=sl)
    torch.cuda.synchronize()
    got = dg.bf16_to_f32(_np(out))
    assert np.isfinite(got).all()
    for b, L in enumerate(lens):
        want = dg.bf16_to_f32(oracle.attention_decode_baseline(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv,
                                                               D, max_seq, L))[0]
        assert _relerr(got[b], want) <= ATTN_TOL, (b, L)


def _prefill_cases():
    rng = np.random.default_rng(0x5EEA)
    cases = []
    for i in range(8):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 4, 8]))
        Hkv = int(rng.choice([1, 2]))
        S = int(rng.integers(1, 300))
        start = int(rng.integers(0, 2500))
        cases.append((i, D, G, Hkv, S, start))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,S,start", _prefill_cases())
def test_sweep_prefill_cached(i, D, G, Hkv, S, start):
    import torch
    import aila_amd
    Hq = Hkv * G
    max_seq = start + S + 5
    seed = 0x5EF0 + i
    print(f"sweep prefill_cached {i}: D={D} G={G} Hkv={Hkv} S={S} start={start}", flush=True)
    q = dg.normal_bf16(seed, 0, (S, Hq * D))
    kc = dg.normal_bf16(seed, 1, (Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (Hkv, max_seq, D))
    kc[:, start + S:] = 0x7FC0
    vc[:, start + S:] = 0x7FC0
    want = dg.bf16_to_f32(oracle.attention_prefill_cached(q, kc, vc, S, start, Hq, Hkv, D, max_seq))
    need = aila_amd.gqa_prefill_cached_workspace_size(S, start, Hq, Hkv, D)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
    dq, dk, dv = _t(q), _t(kc), _t(vc)
    for w in (None, ws):
        got = dg.bf16_to_f32(_np(aila_amd.gqa_prefill_cached(dq, dk, dv, start, Hq, workspace=w)))
        torch.cuda.synchronize()
        assert np.isfinite(got).all()
        assert _relerr(got, want) <= ATTN_TOL, ("split" if w is not None and need else "whole")
