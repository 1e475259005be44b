"""Pins the oracle's batched decode preparation (QK-norm + partial RoPE +
packed q|gate split + K/V append) and sigmoid_mul (oracle/oracle.cpp).

Checks are independent of the oracle's own formulas: numpy fp64
restatements rounded at the reference's rounding points, closed forms of
the sigmoid gate, the composition with the already-pinned head_rms_norm and
apply_rope, per-sequence independence of the batch, and bit-exact copies.
"""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg


def _np_prep_head(x, w, pos, rot, theta, eps):
    """One head: RMSNorm (bf16 round), NeoX rotation of the first `rot` dims
    at `pos` in fp64, bf16 round; dims >= rot keep the normalised value."""
    xf = dg.bf16_to_f32(x).astype(np.float64)
    D = xf.shape[-1]
    rms = np.sqrt((xf ** 2).mean() + eps)
    wf = np.ones(D) if w is None else dg.bf16_to_f32(w).astype(np.float64)
    n = dg.bf16_to_f32(dg.f32_to_bf16((xf / rms * wf).astype(np.float32))).astype(np.float64)
    half = rot // 2
    inv = 1.0 / theta ** (np.arange(half) * 2.0 / rot)
    c, s = np.cos(pos * inv), np.sin(pos * inv)
    out = n.copy()
    out[:half] = n[:half] * c - n[half:rot] * s
    out[half:rot] = n[half:rot] * c + n[:half] * s
    return dg.f32_to_bf16(out.astype(np.float32))


def _close(got, want):
    """bf16 rounding (2^-8 relative) plus the fp32 angle error: the oracle
    forms pos * inv_freq in fp32, which at pos ~3e4 is off by ~2e-3 rad."""
    g = dg.bf16_to_f32(got).astype(np.float64)
    w = dg.bf16_to_f32(want).astype(np.float64)
    return np.all(np.abs(g - w) <= 2 ** -8 * np.abs(w) + 4e-3 * np.abs(w).max())


@pytest.mark.parametrize("D,rot", [(128, 128), (256, 64), (64, 32)])
def test_decode_prepare_vs_numpy(D, rot):
    B, Hq, Hkv, theta, eps = 3, 8, 2, 1e6, 1e-6
    pos = np.array([0, 17, 30000], np.int32)
    q = dg.normal_bf16(501, 0, (B, Hq, D), std=2.0)
    k = dg.normal_bf16(501, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(501, 2, (B, Hkv, D))
    qw = dg.normal_bf16(501, 3, (D,))
    kw = dg.normal_bf16(501, 4, (D,))
    qo, _, ko = oracle.decode_prepare(q, k, v, qw, kw, None, None, pos, B, Hq, Hkv, D, 0, rot, theta, eps)
    for b in range(B):
        for h in range(Hq):
            want = _np_prep_head(q[b, h], qw, float(pos[b]), rot, theta, eps)
            assert _close(qo[b, h], want)
        for h in range(Hkv):
            want = _np_prep_head(k[b, h], kw, float(pos[b]), rot, theta, eps)
            assert _close(ko[b, h], want)


def test_decode_prepare_composes_norm_and_rope():
    """Equals head_rms_norm followed by apply_rope (both pinned elsewhere),
    bit-exact, for a partial rotary width; position 0 rotates nothing."""
    B, Hq, Hkv, D, rot, theta, eps = 2, 4, 2, 256, 64, 1e7, 1e-6
    pos = np.array([0, 1234], np.int32)
    q = dg.normal_bf16(502, 0, (B, Hq, D))
    k = dg.normal_bf16(502, 1, (B, Hkv, D))
    v = dg.normal_bf16(502, 2, (B, Hkv, D))
    qo, _, ko = oracle.decode_prepare(q, k, v, None, None, None, None, pos, B, Hq, Hkv, D, 0, rot, theta, eps)
    for b in range(B):
        qn = oracle.head_rms_norm(q[b].reshape(1, Hq * D), eps, 1, Hq, D)
        kn = oracle.head_rms_norm(k[b].reshape(1, Hkv * D), eps, 1, Hkv, D)
        qr, kr = oracle.apply_rope(qn, kn, 1, int(pos[b]), Hq, Hkv, D, rot, theta)
        assert np.array_equal(qo[b].reshape(1, -1), qr) and np.array_equal(ko[b].reshape(1, -1), kr)
        if pos[b] == 0:
            assert np.array_equal(qr, qn)
        # dims past the rotary width are the normalised values
        assert np.array_equal(qo[b][:, rot:], qn.reshape(Hq, D)[:, rot:])


def test_decode_prepare_packed_gate_and_append():
    B, Hq, Hkv, D, rot, max_seq = 2, 4, 2, 128, 128, 40
    pos = np.array([5, 39], np.int32)
    qg = dg.normal_bf16(503, 0, (B, Hq, 2 * D))
    k = dg.normal_bf16(503, 1, (B, Hkv, D))
    v = dg.normal_bf16(503, 2, (B, Hkv, D))
    kc = dg.normal_bf16(503, 3, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(503, 4, (B, Hkv, max_seq, D))
    kc0, vc0 = kc.copy(), vc.copy()
    qo, gate, ko = oracle.decode_prepare(qg, k, v, None, None, kc, vc, pos, B, Hq, Hkv, D, max_seq, rot,
                                         1e6, 1e-6, packed=True)
    # the gate half is copied through bit-exact; q is the unpacked path
    assert np.array_equal(gate, qg[:, :, D:])
    qo2, _, _ = oracle.decode_prepare(np.ascontiguousarray(qg[:, :, :D]), k, v, None, None, None, None, pos,
                                      B, Hq, Hkv, D, 0, rot, 1e6, 1e-6)
    assert np.array_equal(qo, qo2)
    # appended rows are k_out / v; every other row is untouched
    for b in range(B):
        assert np.array_equal(kc[b, :, pos[b]], ko[b]) and np.array_equal(vc[b, :, pos[b]], v[b])
        mask = np.ones(max_seq, bool)
        mask[pos[b]] = False
        assert np.array_equal(kc[b][:, mask], kc0[b][:, mask]) and np.array_equal(vc[b][:, mask], vc0[b][:, mask])


def test_decode_prepare_batch_is_independent():
    B, Hq, Hkv, D = 3, 4, 4, 64
    pos = np.array([3, 9, 0], np.int32)
    q = dg.normal_bf16(504, 0, (B, Hq, D))
    k = dg.normal_bf16(504, 1, (B, Hkv, D))
    v = dg.normal_bf16(504, 2, (B, Hkv, D))
    qo, _, ko = oracle.decode_prepare(q, k, v, None, None, None, None, pos, B, Hq, Hkv, D, 0, D, 1e6, 1e-6)
    for b in range(B):
        q1, _, k1 = oracle.decode_prepare(q[b:b + 1], k[b:b + 1], v[b:b + 1], None, None, None, None,
                                          pos[b:b + 1], 1, Hq, Hkv, D, 0, D, 1e6, 1e-6)
        assert np.array_equal(qo[b:b + 1], q1) and np.array_equal(ko[b:b + 1], k1)


def test_sigmoid_mul_closed_forms_and_numpy():
    x = dg.normal_bf16(505, 0, (4096,), std=3.0)
    zero = np.zeros(4096, np.uint16)
    # sigmoid(0) = 1/2 exactly: x/2 is exact in bf16 (no subnormals here)
    assert np.array_equal(oracle.sigmoid_mul(x, zero), dg.f32_to_bf16(dg.bf16_to_f32(x) * 0.5))
    # sigmoid(30) rounds to 1 in fp32: the gate is the identity
    big = dg.f32_to_bf16(np.full(4096, 30.0, np.float32))
    assert np.array_equal(oracle.sigmoid_mul(x, big), x)
    g = dg.normal_bf16(505, 1, (4096,), std=4.0)
    want = dg.bf16_to_f32(x).astype(np.float64) / (1.0 + np.exp(-dg.bf16_to_f32(g).astype(np.float64)))
    got = dg.bf16_to_f32(oracle.sigmoid_mul(x, g)).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 2 ** -8 * np.max(np.abs(want))


def test_decode_prepare_with_the_backends_frequency_table():
    """decode_prepare_qkv with rope_freq (ElementwiseOps.cpp:105-216): the
    backends' own table 1/theta^(2d/D) (Qwen3DenseBackend.cpp:232-236) gives
    the theta form bit for bit; an all-zero table rotates nothing (the
    normalised heads); a table scaled by s at position p equals the theta
    form at position s*p when s*p is an integer the float product keeps."""
    Hq, Hkv, D, theta, eps = 8, 2, 128, 1e6, 1e-6
    q = dg.normal_bf16(510, 0, (Hq, D))
    k = dg.normal_bf16(510, 1, (Hkv, D))
    v = dg.normal_bf16(510, 2, (Hkv, D))
    qw = dg.normal_bf16(510, 3, (D,))
    kw = dg.normal_bf16(510, 4, (D,))
    table = np.array([np.float32(1.0) / np.power(np.float32(theta), np.float32(2.0 * d) / np.float32(D),
                                                  dtype=np.float32) for d in range(D // 2)], np.float32)
    # the oracle's theta form computes the same float table
    qa, ka = oracle.decode_prepare_qkv_freq(q, k, v, table, qw, kw, None, None, 777, Hq, Hkv, D, eps, 0)
    qb, _, kb = oracle.decode_prepare(q[None], k[None], v[None], qw, kw, None, None, np.array([777], np.int32), 1,
                                      Hq, Hkv, D, 0, D, theta, eps)
    assert np.array_equal(qa, qb[0]) and np.array_equal(ka, kb[0])
    qz, kz = oracle.decode_prepare_qkv_freq(q, k, v, np.zeros(D // 2, np.float32), qw, kw, None, None, 777, Hq, Hkv,
                                            D, eps, 0)
    assert np.array_equal(qz.reshape(1, -1), oracle.head_rms_norm(q.reshape(1, -1), eps, 1, Hq, D, w_bf16=qw))
    assert np.array_equal(kz.reshape(1, -1), oracle.head_rms_norm(k.reshape(1, -1), eps, 1, Hkv, D, w_bf16=kw))
    qs, ks = oracle.decode_prepare_qkv_freq(q, k, v, table * np.float32(0.5), qw, kw, None, None, 1000, Hq, Hkv, D,
                                            eps, 0)
    qt, _, kt = oracle.decode_prepare(q[None], k[None], v[None], qw, kw, None, None, np.array([500], np.int32), 1,
                                      Hq, Hkv, D, 0, D, theta, eps)
    assert np.array_equal(qs, qt[0]) and np.array_equal(ks, kt[0])
