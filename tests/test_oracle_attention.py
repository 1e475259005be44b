"""Pins the CPU oracle's attention functions (oracle/oracle.cpp).

The reference ships no golden vectors for this path (no kernel tests), so the
oracle is pinned by independent numpy restatements in fp64, closed forms and
invariants, chosen so that a transposed operand, a wrong GQA head mapping, a
dropped scale or an off-by-one causal mask fails at least one test.
"""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg


def _np_attention(q, kc, vc, S, start_pos, Hq, Hkv, D, max_seq):
    """Independent fp64 einsum restatement (softmax(q k^T / sqrt(D)) v)."""
    qf = dg.bf16_to_f32(q).astype(np.float64).reshape(S, Hq, D)
    kf = dg.bf16_to_f32(kc).astype(np.float64).reshape(Hkv, max_seq, D)
    vf = dg.bf16_to_f32(vc).astype(np.float64).reshape(Hkv, max_seq, D)
    g = Hq // Hkv
    out = np.zeros((S, Hq, D))
    for h in range(Hq):
        kh = h // g
        s = qf[:, h, :] @ kf[kh].T / np.sqrt(D)            # [S, max_seq]
        pos = start_pos + np.arange(S)[:, None]
        s = np.where(np.arange(max_seq)[None, :] <= pos, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ vf[kh]
    return out


def _rand_decode(seed, B, Hq, Hkv, D, max_seq):
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    return q, kc, vc


def _relerr(a, r):
    return float(np.max(np.abs(a - r)) / max(np.max(np.abs(r)), 1e-30))


# ------------------------------------------------------------- bf16 -------
def _bf16_by_definition(u32):
    """Nearest bf16 to each fp32 (finite inputs), ties to even, computed from
    the two neighbouring bf16 values in exact fp64 arithmetic."""
    x = u32.view(np.float32).astype(np.float64)
    lo = (u32 & np.uint32(0xFFFF0000))
    hi = lo + np.uint32(0x10000)
    flo = lo.view(np.float32).astype(np.float64)
    fhi = hi.view(np.float32).astype(np.float64)
    # the neighbour above the largest finite bf16 is 2^128 (IEEE overflow rule)
    fhi = np.where(np.isinf(fhi), np.sign(fhi) * 2.0 ** 128, fhi)
    dlo = np.abs(x - flo)
    with np.errstate(invalid="ignore"):
        dhi = np.abs(fhi - x)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (((lo >> 16) & 1) == 1))
    return np.where(pick_hi, hi >> 16, lo >> 16).astype(np.uint16)


def test_bf16_rne_against_definition():
    hi16 = np.arange(0, 1 << 16, dtype=np.uint32)
    fin = (hi16 & 0x7F80) != 0x7F80              # finite upper halves only
    hi16 = hi16[fin]
    lows = np.array([0, 1, 0x3FFF, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xFFFF], np.uint32)
    rng = np.random.default_rng(0)
    lows = np.concatenate([lows, rng.integers(0, 1 << 16, 24, dtype=np.uint32)])
    u = ((hi16[:, None] << 16) | lows[None, :]).reshape(-1).astype(np.uint32)
    want = _bf16_by_definition(u)
    got_np = dg.f32_to_bf16(u.view(np.float32))
    got_c = np.zeros_like(got_np)
    f = np.ascontiguousarray(u.view(np.float32))
    oracle.lib().orc_f32_to_bf16_array(f.ctypes.data, got_c.ctypes.data, f.size)
    assert np.array_equal(got_np, want)
    assert np.array_equal(got_c, want)


def test_bf16_matches_torch():
    import torch
    x = dg.normal(7, 0, 1 << 16) * np.float32(1e3)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(dg.f32_to_bf16(x), t)


# ------------------------------------------------------------ decode -------
@pytest.mark.parametrize("Hq,Hkv,D,L", [(16, 8, 128, 512), (16, 4, 256, 300), (8, 8, 64, 33)])
def test_decode_baseline_vs_numpy_f64(Hq, Hkv, D, L):
    max_seq = L + 7
    q, kc, vc = _rand_decode(11, 1, Hq, Hkv, D, max_seq)
    got = dg.bf16_to_f32(oracle.attention_decode_baseline(q, kc, vc, 1, Hq, Hkv, D, max_seq, L))
    want = _np_attention(q, kc[0], vc[0], 1, L - 1, Hq, Hkv, D, max_seq)
    assert _relerr(got.reshape(Hq, D), want.reshape(Hq, D)) < 8e-3
    truth = oracle.attention_f64(q, kc[0], vc[0], 1, L - 1, Hq, Hkv, D, max_seq)
    assert np.max(np.abs(truth - want)) < 1e-12


def test_decode_single_token_is_v0_exactly():
    Hq, Hkv, D, max_seq = 8, 2, 128, 16
    q, kc, vc = _rand_decode(3, 2, Hq, Hkv, D, max_seq)
    out = oracle.attention_decode_baseline(q, kc, vc, 2, Hq, Hkv, D, max_seq, 1)
    for b in range(2):
        for h in range(Hq):
            assert np.array_equal(out[b, h], vc[b, h // (Hq // Hkv), 0])


def test_decode_identical_keys_give_mean_of_v():
    Hq, Hkv, D, L = 4, 1, 64, 50
    q, kc, vc = _rand_decode(5, 1, Hq, Hkv, D, L)
    kc[:] = kc[:, :, :1, :]
    out = dg.bf16_to_f32(oracle.attention_decode_baseline(q, kc, vc, 1, Hq, Hkv, D, L, L))
    mean = dg.bf16_to_f32(vc[0, 0]).astype(np.float64).mean(axis=0)
    for h in range(Hq):
        assert np.max(np.abs(out[0, h] - mean)) < 2e-2 * np.max(np.abs(mean)) + 1e-3


def test_decode_gqa_equals_replicated_mha():
    Hq, Hkv, D, L = 8, 2, 64, 40
    q, kc, vc = _rand_decode(9, 1, Hq, Hkv, D, L)
    g = Hq // Hkv
    kr = np.repeat(kc, g, axis=1)
    vr = np.repeat(vc, g, axis=1)
    a = oracle.attention_decode_baseline(q, kc, vc, 1, Hq, Hkv, D, L, L)
    b = oracle.attention_decode_baseline(q, kr, vr, 1, Hq, Hq, D, L, L)
    assert np.array_equal(a, b)


def test_decode_ignores_cache_rows_beyond_len():
    Hq, Hkv, D, L, max_seq = 4, 2, 64, 20, 64
    q, kc, vc = _rand_decode(13, 1, Hq, Hkv, D, max_seq)
    a = oracle.attention_decode_baseline(q, kc, vc, 1, Hq, Hkv, D, max_seq, L)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, :, L:] = 0x7F80  # +inf: would poison any read past L
    vc2[:, :, L:] = 0x7F80
    b = oracle.attention_decode_baseline(q, kc2, vc2, 1, Hq, Hkv, D, max_seq, L)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("tile", [1, 7, 64, 128, 1000])
def test_splitk_merge_matches_single_pass(tile):
    B, Hq, Hkv, D, L = 2, 8, 2, 128, 333
    q, kc, vc = _rand_decode(17, B, Hq, Hkv, D, L)
    base = dg.bf16_to_f32(oracle.attention_decode_baseline(q, kc, vc, B, Hq, Hkv, D, L, L))
    sk, part = oracle.attention_decode_splitk(q, kc, vc, B, Hq, Hkv, D, L, L, tile, want_partials=True)
    sk = dg.bf16_to_f32(sk)
    assert _relerr(sk, base) < 8e-3
    # Partial records: m is the tile's max scaled score, l its exp-sum.
    qf = dg.bf16_to_f32(q).astype(np.float64)
    kf = dg.bf16_to_f32(kc).astype(np.float64)
    b, h = 1, 5
    s = kf[b, h // 4, :L] @ qf[b, h] / np.sqrt(D)
    t0 = 0
    np.testing.assert_allclose(part[b, h, 0, 0], s[t0:t0 + tile].max(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(part[b, h, 0, 1],
                               np.exp(s[:tile] - s[:tile].max()).sum(), rtol=1e-4)


# ----------------------------------------------------------- prefill -------
@pytest.mark.parametrize("S,Hq,Hkv,D", [(70, 8, 2, 64), (33, 4, 4, 128), (16, 4, 1, 256)])
def test_prefill_naive_and_online_vs_numpy(S, Hq, Hkv, D):
    q = dg.normal_bf16(21, 0, (S, Hq * D))
    k = dg.normal_bf16(21, 1, (S, Hkv * D))
    v = dg.normal_bf16(21, 2, (S, Hkv * D))
    kc = np.zeros((Hkv, S, D), np.uint16)
    vc = np.zeros((Hkv, S, D), np.uint16)
    oracle.copy_to_cache(k, kc, S, 0, Hkv, D, S)
    oracle.copy_to_cache(v, vc, S, 0, Hkv, D, S)
    want = _np_attention(q, kc, vc, S, 0, Hq, Hkv, D, S).reshape(S, Hq * D)
    for got in (oracle.attention_prefill_naive(q, k, v, S, Hq, Hkv, D),
                oracle.attention_prefill_online(q, k, v, S, Hq, Hkv, D, tile=16)):
        assert _relerr(dg.bf16_to_f32(got), want) < 8e-3
    # causal row 0 attends only key 0: output is v0 exactly
    got = oracle.attention_prefill_naive(q, k, v, S, Hq, Hkv, D)
    for h in range(Hq):
        assert np.array_equal(got[0, h * D:(h + 1) * D], v[0, (h // (Hq // Hkv)) * D:(h // (Hq // Hkv) + 1) * D])


def test_prefill_causality_future_keys_do_not_matter():
    S, Hq, Hkv, D = 40, 4, 2, 64
    q = dg.normal_bf16(23, 0, (S, Hq * D))
    k = dg.normal_bf16(23, 1, (S, Hkv * D))
    v = dg.normal_bf16(23, 2, (S, Hkv * D))
    a = oracle.attention_prefill_naive(q, k, v, S, Hq, Hkv, D)
    k2, v2 = k.copy(), v.copy()
    k2[30:] = dg.normal_bf16(24, 1, (S - 30, Hkv * D))
    v2[30:] = dg.normal_bf16(24, 2, (S - 30, Hkv * D))
    b = oracle.attention_prefill_naive(q, k2, v2, S, Hq, Hkv, D)
    assert np.array_equal(a[:30], b[:30])
    assert not np.array_equal(a[30:], b[30:])


def test_prefill_cached_consistent_with_prefill_and_decode():
    S, Hq, Hkv, D, start, max_seq = 24, 8, 2, 128, 40, 96
    total = start + S
    kc = dg.normal_bf16(29, 1, (Hkv, max_seq, D))
    vc = dg.normal_bf16(29, 2, (Hkv, max_seq, D))
    q = dg.normal_bf16(29, 0, (S, Hq * D))
    want = _np_attention(q, kc, vc, S, start, Hq, Hkv, D, max_seq).reshape(S, Hq * D)
    for online in (False, True):
        got = oracle.attention_prefill_cached(q, kc, vc, S, start, Hq, Hkv, D, max_seq, online)
        assert _relerr(dg.bf16_to_f32(got), want) < 8e-3
    # last query row == decode at cached_len = total
    naive = oracle.attention_prefill_cached(q, kc, vc, S, start, Hq, Hkv, D, max_seq, False)
    dec = oracle.attention_decode_baseline(q[S - 1].reshape(1, Hq, D), kc[None], vc[None], 1,
                                           Hq, Hkv, D, max_seq, total)
    assert np.array_equal(naive[S - 1], dec.reshape(-1))


def test_copy_to_cache_layout():
    S, H, D, start, max_seq = 5, 3, 8, 4, 16
    src = np.arange(S * H * D, dtype=np.uint16).reshape(S, H * D)
    cache = np.zeros((H, max_seq, D), np.uint16)
    oracle.copy_to_cache(src, cache, S, start, H, D, max_seq)
    for s in range(S):
        for h in range(H):
            assert np.array_equal(cache[h, start + s], src[s, h * D:(h + 1) * D])
    assert not cache[:, :start].any() and not cache[:, start + S:].any()


# ------------------------------------------------------ norm and RoPE -------
def test_head_rms_norm_unit_rms():
    S, H, D = 6, 4, 128
    x = dg.normal_bf16(31, 0, (S, H * D), std=3.0)
    y = dg.bf16_to_f32(oracle.head_rms_norm(x, 1e-6, S, H, D)).reshape(S * H, D)
    rms = np.sqrt((y.astype(np.float64) ** 2).mean(axis=1))
    assert np.all(np.abs(rms - 1.0) < 1e-2)
    assert np.array_equal(oracle.head_rms_norm(x, 1e-6, S, H, D), dg.rms_norm_rows_bf16(x, D))
    w = dg.normal_bf16(31, 1, (D,))
    yw = dg.bf16_to_f32(oracle.head_rms_norm(x, 1e-6, S, H, D, w_bf16=w)).reshape(S * H, D)
    np.testing.assert_allclose(yw, y * dg.bf16_to_f32(w)[None], rtol=2e-2, atol=2e-2)


def _np_rope(x, pos, theta, D):
    """HF-style rotate_half RoPE in fp64: x*cos + rotate_half(x)*sin."""
    half = D // 2
    inv = 1.0 / theta ** (np.arange(half) * 2.0 / D)
    ang = pos * inv
    c = np.concatenate([np.cos(ang)] * 2)
    s = np.concatenate([np.sin(ang)] * 2)
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * c + rot * s


def test_rope_properties():
    S, Hq, Hkv, D, theta = 12, 4, 2, 128, 1e6
    q = dg.normal_bf16(37, 0, (S, Hq * D))
    k = dg.normal_bf16(37, 1, (S, Hkv * D))
    q0, k0 = oracle.apply_rope(q, k, S, 0, Hq, Hkv, D, D, theta)
    # position 0 is the identity
    assert np.array_equal(q0[0], q[0]) and np.array_equal(k0[0], k[0])
    qr, kr = oracle.apply_rope(q, k, S, 100, Hq, Hkv, D, D, theta)
    qf = dg.bf16_to_f32(q).astype(np.float64).reshape(S, Hq, D)
    qrf = dg.bf16_to_f32(qr).astype(np.float64).reshape(S, Hq, D)
    for s in range(S):
        want = _np_rope(qf[s], 100 + s, theta, D)
        assert np.max(np.abs(qrf[s] - want)) < 2e-2
        # norm preserved up to bf16 rounding
        np.testing.assert_allclose(np.linalg.norm(qrf[s], axis=-1),
                                   np.linalg.norm(qf[s], axis=-1), rtol=1e-2)
    # q.k depends only on the position difference (checked in fp64 on the
    # unrounded rotation; the oracle's rounding is covered above)
    a = _np_rope(qf[0, 0], 7, theta, D) @ _np_rope(qf[1, 0], 3, theta, D)
    b = _np_rope(qf[0, 0], 104, theta, D) @ _np_rope(qf[1, 0], 100, theta, D)
    assert abs(a - b) < 1e-9 * max(1.0, abs(a))


def test_decode_prepare_matches_separate_ops():
    Hq, Hkv, D, pos, max_seq, theta = 16, 8, 128, 37, 64, 1e6
    q = dg.normal_bf16(41, 0, (1, Hq * D))
    k = dg.normal_bf16(41, 1, (1, Hkv * D))
    v = dg.normal_bf16(41, 2, (1, Hkv * D))
    w1 = dg.f32_to_bf16(np.ones(D, np.float32))
    kc = np.zeros((Hkv, max_seq, D), np.uint16)
    vc = np.zeros((Hkv, max_seq, D), np.uint16)
    qo, ko = oracle.decode_prepare_qkv(q, k, v, w1, w1, kc, vc, pos, Hq, Hkv, D, 1e-6, theta, max_seq)
    qn = oracle.head_rms_norm(q, 1e-6, 1, Hq, D)
    kn = oracle.head_rms_norm(k, 1e-6, 1, Hkv, D)
    qr, kr = oracle.apply_rope(qn, kn, 1, pos, Hq, Hkv, D, D, theta)
    assert np.array_equal(qo, qr) and np.array_equal(ko, kr)
    assert np.array_equal(kc[:, pos], kr.reshape(Hkv, D))
    assert np.array_equal(vc[:, pos], v.reshape(Hkv, D))
