"""GPU parity: batched decode preparation (QK-norm + RoPE + packed q|gate
split + K/V append), prefill head_rms_norm / apply_rope and sigmoid_mul
against the CPU oracle.

Tolerance: bf16 outputs within max relative error 1e-2 of the oracle; the
copied gate half and the appended V rows are bit-exact; untouched cache
rows stay bit-identical.
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


def _relerr(a, r):
    a, r = dg.bf16_to_f32(a).astype(np.float64), dg.bf16_to_f32(r).astype(np.float64)
    return float(np.max(np.abs(a - r)) / max(float(np.max(np.abs(r))), 1e-30))


def _agree(got, want):
    """Max relative error within TOL and nearly every element bit-equal."""
    assert _relerr(got, want) <= TOL
    assert np.mean(got == want) >= 0.9


@pytest.mark.parametrize("B,Hq,Hkv,D,rot,packed,device_pos", [
    (3, 16, 4, 256, 64, True, True),     # Qwen3.5 attention: partial rotary, packed q|gate
    (2, 8, 2, 128, 128, False, False),   # Qwen3: full rotary, q in place
    (2, 4, 4, 64, 64, False, True),
])
def test_decode_prepare(B, Hq, Hkv, D, rot, packed, device_pos):
    import torch
    import aila_amd
    seed = 700 + D
    theta, eps, max_seq = 1e7, 1e-6, 40000
    pos = np.array([0, 17, 32000][:B], np.int32)
    if not device_pos:
        pos[:] = 123
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D if packed else D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    # small caches on the host side of the oracle: only the appended rows matter
    kc_d = torch.zeros((B, Hkv, max_seq, D), dtype=torch.bfloat16, device="cuda")
    vc_d = torch.zeros_like(kc_d)
    kc_d[:, :, 1] = 1.0   # a neighbouring row that must survive
    q_d, k_d = _t(q), _t(k)
    res = aila_amd.decode_prepare_qkv(
        q_d, k_d, _t(v), _t(qw), _t(kw), kc_d, vc_d, pos=int(pos[0]),
        positions=_t(pos) if device_pos else None, rotary_dim=rot, theta=theta, eps=eps, packed_gate=packed)
    torch.cuda.synchronize()
    qo_want, gate_want, ko_want = oracle.decode_prepare(q, k, v, qw, kw, None, None, pos, B, Hq, Hkv, D, 0,
                                                        rot, theta, eps, packed=packed)
    if packed:
        q_got, gate_got = res
        assert np.array_equal(_np(gate_got), gate_want)
        assert np.array_equal(_np(q_d), q), "packed input must not be modified"
    else:
        q_got = res
        assert q_got.data_ptr() == q_d.data_ptr()
    _agree(_np(q_got), qo_want)
    _agree(_np(k_d), ko_want)
    kc_h, vc_h = _np(kc_d), _np(vc_d)
    for b in range(B):
        p = int(pos[b])
        assert np.array_equal(kc_h[b, :, p], _np(k_d)[b]), "cache row must equal the returned k"
        assert np.array_equal(vc_h[b, :, p], v[b])
        if p != 1:
            assert (kc_h[b, :, 1] == 0x3F80).all()
        untouched = np.ones(max_seq, bool)
        untouched[[p, 1]] = False
        assert not vc_h[b][:, untouched].any()


def test_decode_prepare_no_cache_no_weights():
    import torch
    import aila_amd
    B, Hq, Hkv, D = 2, 8, 2, 128
    q = dg.normal_bf16(710, 0, (B, Hq, D))
    k = dg.normal_bf16(710, 1, (B, Hkv, D))
    v = dg.normal_bf16(710, 2, (B, Hkv, D))
    q_d, k_d = _t(q), _t(k)
    aila_amd.decode_prepare_qkv(q_d, k_d, _t(v), pos=5000, rotary_dim=D, theta=1e6)
    torch.cuda.synchronize()
    pos = np.full(B, 5000, np.int32)
    qo, _, ko = oracle.decode_prepare(q, k, v, None, None, None, None, pos, B, Hq, Hkv, D, 0, D, 1e6, 1e-6)
    _agree(_np(q_d), qo)
    _agree(_np(k_d), ko)


@pytest.mark.parametrize("S,H,D,weighted", [(37, 8, 128, True), (5, 16, 256, False), (300, 4, 64, True)])
def test_head_rms_norm(S, H, D, weighted):
    import torch
    import aila_amd
    x = dg.normal_bf16(720 + D, 0, (S, H, D), std=3.0)
    w = dg.normal_bf16(720 + D, 1, (D,)) if weighted else None
    xd = _t(x)
    aila_amd.head_rms_norm(xd, _t(w) if weighted else None, eps=1e-6)
    torch.cuda.synchronize()
    want = oracle.head_rms_norm(x.reshape(S, H * D), 1e-6, S, H, D, w_bf16=w).reshape(S, H, D)
    _agree(_np(xd), want)


@pytest.mark.parametrize("S,Hq,Hkv,D,rot,start", [(50, 8, 2, 256, 64, 1000), (9, 4, 4, 128, 128, 0),
                                                  (130, 2, 1, 64, 32, 70000)])
def test_apply_rope(S, Hq, Hkv, D, rot, start):
    import torch
    import aila_amd
    q = dg.normal_bf16(730 + D, 0, (S, Hq, D))
    k = dg.normal_bf16(730 + D, 1, (S, Hkv, D))
    qd, kd = _t(q), _t(k)
    aila_amd.apply_rope(qd, kd, start_pos=start, rotary_dim=rot, theta=1e7)
    torch.cuda.synchronize()
    qw, kw = oracle.apply_rope(q.reshape(S, -1), k.reshape(S, -1), S, start, Hq, Hkv, D, rot, 1e7)
    _agree(_np(qd), qw.reshape(S, Hq, D))
    _agree(_np(kd), kw.reshape(S, Hkv, D))
    # dims past the rotary width are untouched
    assert np.array_equal(_np(qd)[..., rot:], q[..., rot:])


@pytest.mark.parametrize("n", [1, 7, 1000003])
def test_sigmoid_mul(n):
    import torch
    import aila_amd
    x = dg.normal_bf16(740, 0, (n,), std=3.0)
    g = dg.normal_bf16(740, 1, (n,), std=4.0)
    want = oracle.sigmoid_mul(x, g)
    out = aila_amd.sigmoid_mul(_t(x), _t(g))
    xd = _t(x)
    aila_amd.sigmoid_mul(xd, _t(g), out=xd)    # in place
    torch.cuda.synchronize()
    _agree(_np(out), want)
    assert np.array_equal(_np(out), _np(xd))


@pytest.mark.parametrize("B,Hq,Hkv,D,rot,packed,device_pos,split", [
    (3, 16, 4, 256, 64, True, True, True),     # Qwen3.5 attention layer
    (2, 16, 8, 128, 128, False, False, True),  # Qwen3
    (2, 8, 1, 128, 32, True, True, True),      # narrow rotary, eight heads per group
    (3, 16, 4, 256, 64, True, True, False),    # no workspace: single pass
])
def test_fused_prepare_append_decode(B, Hq, Hkv, D, rot, packed, device_pos, split):
    """One launch (QK-norm + RoPE + append + split-K or single-pass decode)
    against the oracle's prep followed by its attention, and against the
    two-launch path (decode_prepare_qkv + gqa_decode_append)."""
    import torch
    import aila_amd
    seed, theta, eps, max_seq = 760 + D, 1e7, 1e-6, 2048
    pos = np.array([5, 700, 2047][:B], np.int32) if device_pos else np.full(B, 1500, np.int32)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D if packed else D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc = dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D))
    kc_d, vc_d = _t(kc), _t(vc)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda") if split else None
    res = aila_amd.gqa_decode_prepare_append(
        _t(q), _t(k), _t(v), kc_d, vc_d, int(pos.max()), q_norm_w=_t(qw), k_norm_w=_t(kw), rotary_dim=rot,
        theta=theta, eps=eps, packed_gate=packed, positions=_t(pos) if device_pos else None, workspace=ws)
    torch.cuda.synchronize()
    out, gate = res if packed else (res, None)
    # oracle: prep, append, attention per sequence
    qo, gw, ko = oracle.decode_prepare(q, k, v, qw, kw, kc, vc, pos, B, Hq, Hkv, D, max_seq, rot, theta, eps,
                                       packed=packed)
    got = _np(out)
    for b in range(B):
        want = oracle.attention_decode_baseline(qo[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv, D, max_seq,
                                                int(pos[b]) + 1)[0]
        assert _relerr(got[b], want) <= TOL, f"sequence {b}"
    if packed:
        assert np.array_equal(_np(gate), gw)
    kc_h, vc_h = _np(kc_d), _np(vc_d)
    for b in range(B):
        p = int(pos[b])
        assert np.array_equal(vc_h[b, :, p], v[b])
        _agree(kc_h[b, :, p], ko[b])
    # the two-launch path gives the same attention output
    kc2, vc2 = _t(dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))), _t(dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D)))
    q2, k2 = _t(q), _t(k)
    pr = aila_amd.decode_prepare_qkv(q2, k2, _t(v), _t(qw), _t(kw), None, None, pos=int(pos[0]),
                                     positions=_t(pos) if device_pos else None, rotary_dim=rot, theta=theta,
                                     eps=eps, packed_gate=packed)
    q_prep = pr[0] if packed else pr
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out2 = aila_amd.gqa_decode_append(q_prep, k2, _t(v), kc2, vc2, int(pos.max()), workspace=ws,
                                      positions=_t(pos) if device_pos else None)
    torch.cuda.synchronize()
    _agree(got, _np(out2))


@pytest.mark.parametrize("B,Hq,Hkv,D,rot,device_pos,split", [
    (3, 16, 4, 256, 64, True, True),     # Qwen3.5 attention layer, split-K
    (3, 16, 4, 256, 64, True, False),    # single pass
    (2, 8, 1, 128, 32, False, True),
    (1, 8, 8, 64, 64, True, True),       # G = 1, D = 64, first row of the cache (pos 5)
    (3, 16, 2, 128, 128, True, False),   # G = 8 single pass, full rotary
])
def test_fused_prepare_append_decode_gated(B, Hq, Hkv, D, rot, device_pos, split):
    """packed_gate with apply_gate: the gated-attention epilogue
    (out = attention * sigmoid(gate); Qwen35HybridTextBackend's sigmoid_mul
    after the attention, ElementwiseOps.cpp:519-553) inside the fused decode
    launch. Against the oracle's prep + attention + sigmoid_mul, and against
    the ungated fused launch followed by the sigmoid_mul kernel."""
    import torch
    import aila_amd
    seed, theta, eps, max_seq = 790 + D, 1e7, 1e-6, 2048
    pos = np.array([5, 700, 2047][:B], np.int32) if device_pos else np.full(B, 1500, np.int32)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc = dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D))

    def run(apply_gate):
        ws = (torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
              if split else None)
        kc_d, vc_d = _t(kc), _t(vc)
        res = aila_amd.gqa_decode_prepare_append(
            _t(q), _t(k), _t(v), kc_d, vc_d, int(pos.max()), q_norm_w=_t(qw), k_norm_w=_t(kw), rotary_dim=rot,
            theta=theta, eps=eps, packed_gate=True, apply_gate=apply_gate,
            positions=_t(pos) if device_pos else None, workspace=ws)
        torch.cuda.synchronize()
        return res, kc_d, vc_d

    gated, kc_d, vc_d = run(True)
    assert isinstance(gated, torch.Tensor) and tuple(gated.shape) == (B, Hq, D)
    got = _np(gated)
    qo, gw, ko = oracle.decode_prepare(q, k, v, qw, kw, kc, vc, pos, B, Hq, Hkv, D, max_seq, rot, theta, eps,
                                       packed=True)
    for b in range(B):
        att = oracle.attention_decode_baseline(qo[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv, D, max_seq,
                                               int(pos[b]) + 1)[0]
        want = oracle.sigmoid_mul(att, gw[b])
        assert _relerr(got[b], want) <= TOL, f"sequence {b}"
    kc_h, vc_h = _np(kc_d), _np(vc_d)
    for b in range(B):
        p = int(pos[b])
        assert np.array_equal(vc_h[b, :, p], v[b])
        _agree(kc_h[b, :, p], ko[b])
    (plain, gate), _, _ = run(False)
    two_step = aila_amd.sigmoid_mul(plain, gate)
    torch.cuda.synchronize()
    # one bf16 rounding fewer than the two-launch path: at most one ulp apart
    ts = _np(two_step)
    ulps = np.abs(got.astype(np.int32) - ts.astype(np.int32))
    assert np.all((ulps <= 1) | ((got & 0x7FFF) <= 1) & ((ts & 0x7FFF) <= 1))
    assert _relerr(got, ts) <= TOL


def test_apply_gate_needs_packed():
    import aila_amd
    with pytest.raises(ValueError):
        aila_amd.gqa_decode_prepare_append(None, None, None, None, None, 0, apply_gate=True)


# ---- rotary positions past the cache row: text shift and interleaved mRoPE ----
# (ElementwiseOps.cpp:33-103, 555-863; the oracle's position rule is pinned in
# tests/test_oracle_mrope.py)

def _streams(seed, B, P, hi=3000):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, hi, (B, P)).astype(np.int32) for _ in range(3)]


def _rope_pair(streams, plens, deltas, sec, per_seq=True):
    """The same positions as a device record (aila_amd.rope_pos) and as the
    oracle's dict."""
    import aila_amd
    st = streams if per_seq else [s[0] for s in streams]
    dev = aila_amd.rope_pos(pos_t=_t(st[0]), pos_h=_t(st[1]), pos_w=_t(st[2]), sections=sec,
                            prompt_pos_lens=_t(plens), text_pos_deltas=_t(deltas))
    host = dict(pos_t=st[0], pos_h=st[1], pos_w=st[2], sections=sec, prompt_lens=plens, deltas=deltas)
    return dev, host


@pytest.mark.parametrize("B,Hq,Hkv,D,rot,packed", [
    (3, 16, 4, 256, 64, True),     # Qwen3.5 attention: partial rotary, packed q|gate
    (3, 8, 2, 128, 128, False),
])
def test_decode_prepare_mrope(B, Hq, Hkv, D, rot, packed):
    import torch
    import aila_amd
    seed, theta, eps, max_seq, P = 1700 + D, 1e7, 1e-6, 4096, 600
    sec = (11, 11, 10) if rot == 64 else (24, 20, 20)
    pos = np.array([300, 700, 4000], np.int32)
    plens = np.array([P, 600, 0], np.int32)      # seq 0 inside its prompt, 1 and 2 past it
    deltas = np.array([-100, -250, 9], np.int32)
    dev, host = _rope_pair(_streams(seed, B, P), plens, deltas, sec)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D if packed else D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc_d = torch.zeros((B, Hkv, max_seq, D), dtype=torch.bfloat16, device="cuda")
    vc_d = torch.zeros_like(kc_d)
    k_d = _t(k)
    res = aila_amd.decode_prepare_qkv(_t(q), k_d, _t(v), _t(qw), _t(kw), kc_d, vc_d, positions=_t(pos),
                                      rotary_dim=rot, theta=theta, eps=eps, packed_gate=packed, rope=dev)
    torch.cuda.synchronize()
    q_got = res[0] if packed else res
    qo, _, ko = oracle.decode_prepare(q, k, v, qw, kw, None, None, pos, B, Hq, Hkv, D, 0, rot, theta, eps,
                                      packed=packed, rope=host)
    _agree(_np(q_got), qo)
    _agree(_np(k_d), ko)
    # the rotation moved but the cache row did not
    kc_h = _np(kc_d)
    for b in range(B):
        assert np.array_equal(kc_h[b, :, pos[b]], _np(k_d)[b])
    assert int((kc_h != 0).any(axis=-1).sum()) == B * Hkv
    # and it differs from a plain prep at the row (the positions matter)
    plain = oracle.decode_prepare(q, k, v, qw, kw, None, None, pos, B, Hq, Hkv, D, 0, rot, theta, eps,
                                  packed=packed)[0]
    assert not np.array_equal(plain, qo)


@pytest.mark.parametrize("S,Hq,Hkv,D,rot,start,P,delta", [
    (80, 8, 2, 256, 64, 0, 50, -20),      # a prompt with image positions, then text
    (33, 4, 4, 128, 128, 100, 120, 5),
    (20, 2, 1, 64, 32, 500, 100, 1000),   # a later turn: every row past the prompt
])
def test_apply_rope_mrope(S, Hq, Hkv, D, rot, start, P, delta):
    import torch
    import aila_amd
    sec = (rot // 6, rot // 6, rot // 2 - 2 * (rot // 6))
    st = _streams(1800 + D, 1, P, hi=500)
    q = dg.normal_bf16(1800 + D, 0, (S, Hq, D))
    k = dg.normal_bf16(1800 + D, 1, (S, Hkv, D))
    dev = aila_amd.rope_pos(prompt_pos_len=P, text_pos_delta=delta, pos_t=_t(st[0][0]), pos_h=_t(st[1][0]),
                            pos_w=_t(st[2][0]), sections=sec)
    qd, kd = _t(q), _t(k)
    aila_amd.apply_rope(qd, kd, start_pos=start, rotary_dim=rot, theta=1e6, rope=dev)
    torch.cuda.synchronize()
    host = dict(pos_t=st[0][0], pos_h=st[1][0], pos_w=st[2][0], prompt_pos_len=P, text_pos_delta=delta,
                sections=sec)
    qw, kw = oracle.apply_rope(q.reshape(S, -1), k.reshape(S, -1), S, start, Hq, Hkv, D, rot, 1e6, rope=host)
    _agree(_np(qd), qw.reshape(S, Hq, D))
    _agree(_np(kd), kw.reshape(S, Hkv, D))
    assert np.array_equal(_np(qd)[..., rot:], q[..., rot:])


@pytest.mark.parametrize("apply_gate,split", [(True, True), (False, True), (True, False)])
def test_fused_prepare_append_decode_mrope(apply_gate, split):
    """The one-launch prep + append + decode with shifted / mRoPE positions
    (the hybrid backend's decode after a multimodal prompt,
    Qwen35HybridTextBackend.cpp:2109-2135) against the oracle's prep at those
    positions followed by its attention over rows [0, pos]."""
    import torch
    import aila_amd
    B, Hq, Hkv, D, rot, max_seq, P = 3, 16, 4, 256, 64, 2048, 900
    seed, theta, eps = 1900, 1e7, 1e-6
    sec = (11, 11, 10)
    pos = np.array([400, 1200, 2047], np.int32)
    plens = np.array([P, P, 0], np.int32)
    deltas = np.array([-300, -600, 17], np.int32)
    dev, host = _rope_pair(_streams(seed, B, P), plens, deltas, sec)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc = dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D))
    kc_d, vc_d = _t(kc), _t(vc)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda") if split else None
    res = aila_amd.gqa_decode_prepare_append(
        _t(q), _t(k), _t(v), kc_d, vc_d, int(pos.max()), q_norm_w=_t(qw), k_norm_w=_t(kw), rotary_dim=rot,
        theta=theta, eps=eps, packed_gate=True, apply_gate=apply_gate, positions=_t(pos), workspace=ws, rope=dev)
    torch.cuda.synchronize()
    out = res if apply_gate else res[0]
    qo, gw, ko = oracle.decode_prepare(q, k, v, qw, kw, kc, vc, pos, B, Hq, Hkv, D, max_seq, rot, theta, eps,
                                       packed=True, rope=host)
    got = _np(out)
    for b in range(B):
        want = oracle.attention_decode_baseline(qo[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv, D, max_seq,
                                                int(pos[b]) + 1)[0]
        if apply_gate:
            want = oracle.sigmoid_mul(want, gw[b])
        assert _relerr(got[b], want) <= TOL, f"sequence {b}"
    kc_h = _np(kc_d)
    for b in range(B):
        _agree(kc_h[b, :, pos[b]], ko[b])


def test_decode_prepare_with_a_frequency_table():
    """ops::decode_prepare_qkv's rope_freq table (angle = start_pos *
    rope_freq[d], ElementwiseOps.cpp:105-216) passed as rope_pos.inv_freq,
    with a table that is not theta's (position-interpolated low
    frequencies), in the decode prep and in the one-launch prep + decode."""
    import torch
    import aila_amd
    Hq, Hkv, D, theta, eps, max_seq, pos = 16, 4, 128, 1e6, 1e-6, 2048, 1500
    table = (1.0 / theta ** (np.arange(D // 2) * 2.0 / D)).astype(np.float32)
    table[D // 4:] *= 0.125
    q = dg.normal_bf16(1950, 0, (1, Hq, D), std=2.0)
    k = dg.normal_bf16(1950, 1, (1, Hkv, D), std=2.0)
    v = dg.normal_bf16(1950, 2, (1, Hkv, D))
    qw = dg.normal_bf16(1950, 3, (D,))
    kw = dg.normal_bf16(1950, 4, (D,))
    dev = aila_amd.rope_pos(inv_freq=_t(table))
    q_d, k_d = _t(q), _t(k)
    aila_amd.decode_prepare_qkv(q_d, k_d, _t(v), _t(qw), _t(kw), pos=pos, rotary_dim=D, theta=theta, eps=eps,
                                rope=dev)
    torch.cuda.synchronize()
    qo, ko = oracle.decode_prepare_qkv_freq(q[0], k[0], v[0], table, qw, kw, None, None, pos, Hq, Hkv, D, eps, 0)
    _agree(_np(q_d)[0], qo)
    _agree(_np(k_d)[0], ko)
    # the fused launch with the same table
    kc = dg.normal_bf16(1950, 5, (1, Hkv, max_seq, D))
    vc = dg.normal_bf16(1950, 6, (1, Hkv, max_seq, D))
    kc_d, vc_d = _t(kc), _t(vc)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(1, Hq, D), dtype=torch.uint8, device="cuda")
    out = aila_amd.gqa_decode_prepare_append(_t(q), _t(k), _t(v), kc_d, vc_d, pos, q_norm_w=_t(qw), k_norm_w=_t(kw),
                                             rotary_dim=D, theta=theta, eps=eps, workspace=ws, rope=dev)
    torch.cuda.synchronize()
    kc2, vc2 = kc.copy(), vc.copy()
    qo2, _ = oracle.decode_prepare_qkv_freq(q[0], k[0], v[0], table, qw, kw, kc2[0], vc2[0], pos, Hq, Hkv, D, eps,
                                            max_seq)
    want = oracle.attention_decode_baseline(qo2[None], kc2, vc2, 1, Hq, Hkv, D, max_seq, pos + 1)
    assert _relerr(_np(out), want) <= TOL
    _agree(_np(kc_d)[0, :, pos], kc2[0, :, pos])


def test_fused_decode_first_chunk_waits_for_its_dma():
    """The wave whose first K chunk holds the appended row issues that
    chunk's LDS DMA after the append, just before the loop that reads it; the
    kernel waits for it explicitly (without the wait the G = 8 fused kernel
    read the stage before it landed, now and then, and scored stale LDS).
    Split 23 of 24 is that split here (1501 rows in 64-row splits). Every
    split record is checked against float64 attention over its rows, on
    repeated launches."""
    import torch
    import aila_amd
    B, Hq, Hkv, D, rot = 2, 8, 1, 128, 32
    seed, theta, eps, max_seq, p = 918, 1e7, 1e-6, 2048, 1500
    pos = np.full(B, p, np.int32)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc0 = dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))
    vc0 = dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D))
    kc, vc = kc0.copy(), vc0.copy()
    qo, gw, _ = oracle.decode_prepare(q, k, v, qw, kw, kc, vc, pos, B, Hq, Hkv, D, max_seq, rot, theta, eps,
                                      packed=True)
    f64 = lambda x: dg.bf16_to_f32(x).astype(np.float64)
    wsb = aila_amd.gqa_decode_workspace_size(B, Hq, D)
    nmax = wsb // (B * Hq * (16 + D) * 4)
    want_out = [oracle.attention_decode_baseline(qo[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv, D, max_seq,
                                                 p + 1)[0] for b in range(B)]
    for rep in range(24):
        # fresh host uploads each launch: the cache rows are not in L2, so
        # the K DMA is slow to land (the case the wait is for)
        ws = torch.full((wsb // 4,), float("nan"), dtype=torch.float32, device="cuda")
        out, _ = aila_amd.gqa_decode_prepare_append(_t(q), _t(k), _t(v), _t(kc0), _t(vc0), p, q_norm_w=_t(qw),
                                                    k_norm_w=_t(kw), rotary_dim=rot, theta=theta, eps=eps,
                                                    packed_gate=True, workspace=ws.view(torch.uint8))
        torch.cuda.synchronize()
        rec = ws.cpu().numpy().reshape(B, Hq, nmax, 16 + D)
        ns = int(np.sum(np.isfinite(rec[0, 0, :, 1])))
        assert ns == 24, ns
        got = _np(out)
        for b in range(B):
            assert _relerr(got[b], want_out[b]) <= TOL, f"launch {rep} sequence {b}"
            Kb, Vb = f64(kc[b, 0, :p + 1]), f64(vc[b, 0, :p + 1])
            S = f64(qo[b]) @ Kb.T / np.sqrt(D)
            for i in range(ns):
                s0, s1 = 64 * i, min(64 * i + 64, p + 1)
                m = S[:, s0:s1].max(axis=1, keepdims=True)
                w = np.exp(S[:, s0:s1] - m)
                want = (w @ Vb[s0:s1]) / w.sum(axis=1, keepdims=True)
                r = rec[b, :, i].astype(np.float64)
                np.testing.assert_allclose(r[:, 0], m[:, 0], rtol=1e-3, atol=1e-3,
                                           err_msg=f"launch {rep} sequence {b} split {i} max")
                err = np.abs(r[:, 16:] / r[:, 1:2] - want).max() / np.abs(want).max()
                assert err <= 2e-2, f"launch {rep} sequence {b} split {i}: {err}"


def _close(got, want):
    """Rotations at long positions: at least 99% of the elements bit-equal
    (the frequencies, angles and products are the oracle's floats; cos/sin
    may differ in the last bit and flip a rounding) and the rest within the
    path's tolerance. With the device powf's frequencies 1.3-9% of the
    elements differed at position 1048575."""
    assert _relerr(got, want) <= TOL
    assert np.mean(got == want) >= 0.99


@pytest.mark.parametrize("D,rot,theta", [(128, 128, 1e6), (256, 64, 1e7), (64, 64, 1e4)])
def test_rope_at_long_positions(D, rot, theta):
    """Positions up to 2^20 (ElementwiseOps.cpp:80-83: angle = position *
    1/pow(theta, 2d/rot)). The inverse frequencies are the correctly rounded
    floats of that formula; with the device powf (not correctly rounded) a
    frequency one ulp off turned the angle by position * ulp, ~3e-2 relative
    error at position 1M."""
    import torch
    import aila_amd
    B, Hq, Hkv = 3, 8, 2
    pos = np.array([65535, 262143, 1048575], np.int32)
    q = dg.normal_bf16(740 + D, 0, (B, Hq, D))
    k = dg.normal_bf16(740 + D, 1, (B, Hkv, D))
    v = dg.normal_bf16(740 + D, 2, (B, Hkv, D))
    q_d, k_d = _t(q), _t(k)
    aila_amd.decode_prepare_qkv(q_d, k_d, _t(v), positions=_t(pos), rotary_dim=rot, theta=theta)
    torch.cuda.synchronize()
    qo, _, ko = oracle.decode_prepare(q, k, v, None, None, None, None, pos, B, Hq, Hkv, D, 0, rot, theta, 1e-6)
    _close(_np(q_d), qo)
    _close(_np(k_d), ko)
    # prefill rows at the same range of positions
    S, start = 6, 1048570
    qs = dg.normal_bf16(741 + D, 0, (S, Hq, D))
    ks = dg.normal_bf16(741 + D, 1, (S, Hkv, D))
    qsd, ksd = _t(qs), _t(ks)
    aila_amd.apply_rope(qsd, ksd, start_pos=start, rotary_dim=rot, theta=theta)
    torch.cuda.synchronize()
    qw, kw = oracle.apply_rope(qs.reshape(S, -1), ks.reshape(S, -1), S, start, Hq, Hkv, D, rot, theta)
    _close(_np(qsd), qw.reshape(S, Hq, D))
    _close(_np(ksd), kw.reshape(S, Hkv, D))


def test_fused_prepare_append_decode_long_position():
    """The one-launch prep + append + decode at cache row 262143 (a 256k
    context, Qwen3.5 attention shape): the appended, rotated k row against
    the oracle's prep, and the attention over all 262144 rows."""
    import torch
    import aila_amd
    B, Hq, Hkv, D, rot, theta, eps = 1, 4, 1, 256, 64, 1e7, 1e-6
    pos = np.array([262143], np.int32)
    max_seq = 262144
    seed = 750
    print(f"fused prep long position pos={pos[0]} max_seq={max_seq}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc = dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D))
    kc_d, vc_d = _t(kc), _t(vc)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out, gate = aila_amd.gqa_decode_prepare_append(
        _t(q), _t(k), _t(v), kc_d, vc_d, int(pos[0]), q_norm_w=_t(qw), k_norm_w=_t(kw), rotary_dim=rot,
        theta=theta, eps=eps, packed_gate=True, positions=_t(pos), workspace=ws)
    torch.cuda.synchronize()
    qo, gw, ko = oracle.decode_prepare(q, k, v, qw, kw, kc, vc, pos, B, Hq, Hkv, D, max_seq, rot, theta, eps,
                                       packed=True)
    _close(_np(kc_d)[0, :, pos[0]], ko[0])
    assert np.array_equal(_np(vc_d)[0, :, pos[0]], v[0])
    assert np.array_equal(_np(gate), gw)
    want = oracle.attention_decode_baseline(qo, kc, vc, 1, Hq, Hkv, D, max_seq, int(pos[0]) + 1)[0]
    assert _relerr(_np(out)[0], want) <= TOL


def test_apply_rope_prompt_past_65535_tokens():
    """A 100000-token prompt through apply_rope (tokens on the grid's x axis,
    so no 65535-token cap): every row against the oracle."""
    import torch
    import aila_amd
    S, Hq, Hkv, D, rot, start = 100000, 2, 1, 64, 64, 7
    q = dg.normal_bf16(745, 0, (S, Hq, D))
    k = dg.normal_bf16(745, 1, (S, Hkv, D))
    qd, kd = _t(q), _t(k)
    aila_amd.apply_rope(qd, kd, start_pos=start, rotary_dim=rot, theta=1e6)
    torch.cuda.synchronize()
    qw, kw = oracle.apply_rope(q.reshape(S, -1), k.reshape(S, -1), S, start, Hq, Hkv, D, rot, 1e6)
    _close(_np(qd), qw.reshape(S, Hq, D))
    _close(_np(kd), kw.reshape(S, Hkv, D))
