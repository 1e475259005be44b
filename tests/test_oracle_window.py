"""Pins the oracle's decode window with attention sinks
(orc_attention_decode_window: ops::attention_decode's
AILA_ATTN_DECODE_WINDOW / _WINDOW_START / _SINK plan, AttentionOps.cpp:
533-551, 598-616, on the baseline kernel's row map :73-166).

Each case reduces to the already-pinned full-context decode: attending rows
[0, s) and [L - w, L) equals the plain decode over a cache holding exactly
those rows, in that order (bit-exact: the same sums in the same order), and
every way the window switches off (window 0, L <= window_start, sink and
tail meeting) is the plain decode itself. An fp64 masked softmax checks one
case independently.
"""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg


def _case(seed, Hq=8, Hkv=2, D=128, max_seq=1500):
    q = dg.normal_bf16(seed, 0, (1, Hq, D))
    kc = dg.normal_bf16(seed, 1, (1, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (1, Hkv, max_seq, D))
    return q, kc, vc


def _plain_over_rows(q, kc, vc, rows, Hq, Hkv, D):
    k2 = np.ascontiguousarray(kc[:, :, rows])
    v2 = np.ascontiguousarray(vc[:, :, rows])
    return oracle.attention_decode_baseline(q, k2, v2, 1, Hq, Hkv, D, len(rows), len(rows))


@pytest.mark.parametrize("L,window,start,sink", [
    (1200, 256, 512, 0),      # tail only
    (1200, 256, 512, 5),      # sink of 5 rows (not a chunk multiple)
    (1300, 700, -1, 64),      # default start = max(512, window) = 700
])
def test_window_equals_plain_decode_over_the_kept_rows(L, window, start, sink):
    Hq, Hkv, D = 8, 2, 128
    q, kc, vc = _case(950)
    got = oracle.attention_decode_window(q, kc, vc, 1, Hq, Hkv, D, 1500, L, window, start, sink)
    rows = list(range(min(sink, L - window))) + list(range(L - window, L))
    want = _plain_over_rows(q, kc, vc, rows, Hq, Hkv, D)
    assert np.array_equal(got, want)
    full = oracle.attention_decode_baseline(q, kc, vc, 1, Hq, Hkv, D, 1500, L)
    assert not np.array_equal(got, full), "the window must change the result"


@pytest.mark.parametrize("L,window,start,sink", [
    (1200, 0, 512, 8),        # window off
    (500, 256, 512, 8),       # not longer than window_start
    (600, 400, 512, 300),     # sink and tail meet: whole context
    (700, 700, 512, 0),       # window covers everything
])
def test_window_off_is_plain_decode(L, window, start, sink):
    Hq, Hkv, D = 8, 2, 128
    q, kc, vc = _case(951)
    got = oracle.attention_decode_window(q, kc, vc, 1, Hq, Hkv, D, 1500, L, window, start, sink)
    assert np.array_equal(got, oracle.attention_decode_baseline(q, kc, vc, 1, Hq, Hkv, D, 1500, L))


def test_window_fp64_masked_softmax_and_per_sequence_lengths():
    B, Hq, Hkv, D, max_seq = 3, 4, 2, 64, 900
    q = dg.normal_bf16(952, 0, (B, Hq, D))
    kc = dg.normal_bf16(952, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(952, 2, (B, Hkv, max_seq, D))
    lens = np.array([900, 300, 700], np.int32)
    window, start, sink = 200, 512, 3
    got = oracle.attention_decode_window(q, kc, vc, B, Hq, Hkv, D, max_seq, 900, window, start, sink, lens=lens)
    for b in range(B):
        L = int(lens[b])
        keep = np.zeros(L, bool)
        if L > start:
            keep[:sink] = True
            keep[L - window:] = True
        else:
            keep[:] = True
        qf = dg.bf16_to_f32(q[b]).astype(np.float64)
        kf = dg.bf16_to_f32(kc[b, :, :L]).astype(np.float64)
        vf = dg.bf16_to_f32(vc[b, :, :L]).astype(np.float64)
        for h in range(Hq):
            g = h // (Hq // Hkv)
            s = kf[g] @ qf[h] / np.sqrt(D)
            s[~keep] = -np.inf
            p = np.exp(s - s.max())
            p /= p.sum()
            want = p @ vf[g]
            o = dg.bf16_to_f32(got[b, h]).astype(np.float64)
            assert np.max(np.abs(o - want)) <= 1e-2 * np.max(np.abs(want)) + 1e-6
