"""Seeded sweeps of GPU parity over shapes and lengths the targeted tests do
not pin one by one, each case checked against the CPU oracle:
  - split-K decode with device-side lengths (each sequence's rows shared
    evenly by the launched splits), AttentionOps.cpp:73-320;
  - prefill over a cached prefix with and without the key split, :2308-2507;
  - causal prefill with the fused cache write, :649-842 and :2513-2532;
  - chunked and recurrent DeltaNet, Qwen35HybridTextBackend.cpp:1729-1780;
  - paged decode (bit-exact against the contiguous decode of the same rows);
  - the fused decode preparation + append + decode at device positions;
  - the whole DeltaNet layer, prefill then decode steps.
Attention outputs within max relative error 1e-2, DeltaNet states within
1e-3; cache rows and pool pages past the attended range hold NaN.

AILA_SWEEP_SEED=n draws another set of cases (default 0: the set the suite
runs by default); a range "a-b" or a list "a,b,c" runs the sets of several
seeds in one process."""
import os

import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg

pytestmark = pytest.mark.gpu
ATTN_TOL = 1e-2


def _parse_seeds(text):
    seeds = []
    for part in text.split(","):
        part = part.strip()
        if "-" in part:
            lo, hi = (int(x) for x in part.split("-", 1))
            seeds.extend(range(lo, hi + 1))
        elif part:
            seeds.append(int(part))
    return seeds or [0]


SWEEP_SEEDS = _parse_seeds(os.environ.get("AILA_SWEEP_SEED", "0"))


def _all(gen):
    return [case for seed in SWEEP_SEEDS for case in gen(seed)]


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


def _decode_cases(sweep_seed):
    rng = np.random.default_rng(0x5EE9 + sweep_seed)
    cases = []
    for i in range(16):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
        Hkv = int(rng.choice([1, 2, 4]))
        B = int(rng.integers(1, 6))
        bound = int(rng.integers(64, 3000))
        lens = [int(x) for x in rng.integers(1, bound + 1, size=B)]
        lens[0] = min(lens[0], int(rng.choice([1, 15, 16, 17])))   # short sequences beside long ones
        cases.append((i, D, G, Hkv, B, bound, lens))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,B,bound,lens", _all(_decode_cases))
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


def _prefill_cases(sweep_seed):
    rng = np.random.default_rng(0x5EEA + sweep_seed)
    cases = []
    for i in range(16):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
        Hkv = int(rng.choice([1, 2]))
        S = int(rng.integers(1, 300))
        start = int(rng.integers(0, 2500))
        cases.append((i, D, G, Hkv, S, start))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,S,start", _all(_prefill_cases))
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


def _prefill_uncached_cases(sweep_seed):
    rng = np.random.default_rng(0x5EEB + sweep_seed)
    cases = []
    for i in range(12):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
        Hkv = int(rng.choice([1, 2]))
        S = int(rng.integers(1, 700))
        cache_pos = int(rng.integers(0, 50))
        cases.append((i, D, G, Hkv, S, cache_pos))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,S,cache_pos", _all(_prefill_uncached_cases))
def test_sweep_prefill_with_cache_write(i, D, G, Hkv, S, cache_pos):
    """Causal prefill (AttentionOps.cpp:649-842) with the fused cache write
    (copy_to_cache, :2513-2532): output within tolerance, cache bit-exact."""
    import torch
    import aila_amd
    Hq = Hkv * G
    seed = 0x5F00 + i
    print(f"sweep prefill {i}: D={D} G={G} Hkv={Hkv} S={S} cache_pos={cache_pos}", flush=True)
    q = dg.normal_bf16(seed, 0, (S, Hq * D))
    k = dg.normal_bf16(seed, 1, (S, Hkv * D))
    v = dg.normal_bf16(seed, 2, (S, Hkv * D))
    max_seq = cache_pos + S + 3
    kc = torch.full((Hkv, max_seq, D), 5.0, dtype=torch.bfloat16, device="cuda")
    vc = torch.full((Hkv, max_seq, D), 5.0, dtype=torch.bfloat16, device="cuda")
    out = aila_amd.gqa_prefill(_t(q), _t(k), _t(v), Hq, Hkv, k_cache=kc, v_cache=vc, cache_pos=cache_pos)
    torch.cuda.synchronize()
    got = dg.bf16_to_f32(_np(out))
    want = dg.bf16_to_f32(oracle.attention_prefill_naive(q, k, v, S, Hq, Hkv, D))
    assert np.isfinite(got).all()
    assert _relerr(got, want) <= ATTN_TOL
    ck = np.full((Hkv, max_seq, D), dg.f32_to_bf16(np.float32([5.0]))[0], np.uint16)
    cv = ck.copy()
    oracle.copy_to_cache(k, ck, S, cache_pos, Hkv, D, max_seq)
    oracle.copy_to_cache(v, cv, S, cache_pos, Hkv, D, max_seq)
    assert np.array_equal(_np(kc), ck) and np.array_equal(_np(vc), cv)


def _deltanet_prefill_cases(sweep_seed):
    rng = np.random.default_rng(0x5EEC + sweep_seed)
    cases = []
    for i in range(12):
        B = int(rng.integers(1, 4))
        T = int(rng.integers(1, 400))
        Hk = int(rng.choice([1, 2, 4]))
        ratio = int(rng.choice([1, 2, 4]))
        gates = bool(rng.integers(0, 2))
        s0 = float(rng.choice([0.0, 0.02]))
        cases.append((i, B, T, Hk, Hk * ratio, gates, s0))
    return cases


@pytest.mark.parametrize("i,B,T,Hk,Hv,gates,s0", _all(_deltanet_prefill_cases))
def test_sweep_deltanet_prefill(i, B, T, Hk, Hv, gates, s0):
    """Chunked prefill against the sequential recurrence
    (Qwen35HybridTextBackend.cpp:1729-1780): outputs 1e-2, state 1e-3."""
    import torch
    import aila_amd
    d = 128
    seed = 0x5F10 + i
    print(f"sweep deltanet prefill {i}: B={B} T={T} Hk={Hk} Hv={Hv} gates={gates} s0={s0}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, T, Hk, d))
    k = dg.normal_bf16(seed, 1, (B, T, Hk, d))
    v = dg.normal_bf16(seed, 2, (B, T, Hv, d))
    a = dg.normal_bf16(seed, 3, (B, T, Hv))
    b = dg.normal_bf16(seed, 4, (B, T, Hv))
    S0 = (dg.normal(seed, 5, B * Hv * d * d, std=s0).reshape(B, Hv, d, d) if s0 > 0
          else np.zeros((B, Hv, d, d), np.float32)).astype(np.float32)
    dtb = dg.normal_bf16(seed, 6, (Hv,), std=0.5) if gates else None
    alog = dg.normal(seed, 7, Hv, std=0.3).astype(np.float32) if gates else None
    st = _t(S0)
    out = aila_amd.deltanet_prefill(_t(q), _t(k), _t(v), _t(a), _t(b), st,
                                    dt_bias=_t(dtb) if gates else None, A_log=_t(alog) if gates else None)
    torch.cuda.synchronize()
    _, want_ob, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T, Hk, Hv, d, d, dt_bias=dtb, A_log=alog)
    got_o, got_S = dg.bf16_to_f32(_np(out)), st.cpu().numpy()
    assert np.isfinite(got_o).all() and np.isfinite(got_S).all()
    assert _relerr(got_o, dg.bf16_to_f32(want_ob)) <= ATTN_TOL
    assert _relerr(got_S, want_S) <= 1e-3


def _deltanet_decode_cases(sweep_seed):
    rng = np.random.default_rng(0x5EED + sweep_seed)
    cases = []
    for i in range(12):
        dk = int(rng.choice([64, 128, 256]))
        dv = int(rng.choice([64, 128, 200, 256]))
        Hk = int(rng.choice([1, 2, 8, 16]))
        Hv = Hk * int(rng.choice([1, 2]))
        B = int(rng.choice([1, 3, 16, 40]))    # both sides of the wide-slab threshold
        cases.append((i, B, Hk, Hv, dk, dv))
    return cases


@pytest.mark.parametrize("i,B,Hk,Hv,dk,dv", _all(_deltanet_decode_cases))
def test_sweep_deltanet_decode(i, B, Hk, Hv, dk, dv):
    """Recurrent decode steps (Qwen35HybridTextBackend.cpp:1094-1148) against
    the sequential oracle over 4 steps."""
    import torch
    import aila_amd
    T = 4
    seed = 0x5F20 + i
    print(f"sweep deltanet decode {i}: B={B} Hk={Hk} Hv={Hv} dk={dk} dv={dv}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, T, Hk, dk))
    k = dg.normal_bf16(seed, 1, (B, T, Hk, dk))
    v = dg.normal_bf16(seed, 2, (B, T, Hv, dv))
    a = dg.normal_bf16(seed, 3, (B, T, Hv))
    b = dg.normal_bf16(seed, 4, (B, T, Hv))
    S0 = dg.normal(seed, 5, B * Hv * dk * dv, std=0.02).reshape(B, Hv, dk, dv).astype(np.float32)
    st = _t(S0)
    dq, dkk, dvv, da, db = (_t(np.ascontiguousarray(x)) for x in (q, k, v, a, b))
    outs = [aila_amd.deltanet_decode(dq[:, t].contiguous(), dkk[:, t].contiguous(), dvv[:, t].contiguous(),
                                     da[:, t].contiguous(), db[:, t].contiguous(), st) for t in range(T)]
    torch.cuda.synchronize()
    got_o = dg.bf16_to_f32(np.stack([_np(o) for o in outs], axis=1))
    _, want_ob, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T, Hk, Hv, dk, dv)
    assert _relerr(st.cpu().numpy(), want_S) <= 1e-3
    assert _relerr(got_o, dg.bf16_to_f32(want_ob)) <= ATTN_TOL


def _paged_cases(sweep_seed):
    rng = np.random.default_rng(0x5EEE + sweep_seed)
    cases = []
    for i in range(12):
        page = int(rng.choice([16, 32, 48, 64, 128, 256]))
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
        B = int(rng.integers(1, 5))
        max_pages = int(rng.integers(2, 12))
        lens = [int(x) for x in rng.integers(1, page * max_pages + 1, size=B)]
        cases.append((i, page, D, G, B, max_pages, lens))
    return cases


@pytest.mark.parametrize("i,page,D,G,B,max_pages,lens", _all(_paged_cases))
def test_sweep_paged_decode(i, page, D, G, B, max_pages, lens):
    """Paged decode equals the contiguous decode of the same rows bit for
    bit and the oracle within tolerance; unowned pool pages hold NaN."""
    import torch
    import aila_amd
    Hkv = 2
    Hq = Hkv * G
    max_seq = page * max_pages
    seed = 0x5F30 + i
    print(f"sweep paged {i}: page={page} D={D} G={G} B={B} max_pages={max_pages} lens={lens}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    for b, L in enumerate(lens):
        kc[b, :, L:] = 0x7FC0
        vc[b, :, L:] = 0x7FC0
    npages = B * max_pages + 3
    perm = np.random.default_rng(seed).permutation(npages)
    pk = np.full((npages, Hkv, page, D), 0x7FC0, np.uint16)
    pv = pk.copy()
    table = np.zeros((B, max_pages), np.int32)
    for b in range(B):
        for j in range(max_pages):
            p = int(perm[b * max_pages + j])
            table[b, j] = p
            pk[p] = kc[b, :, j * page:(j + 1) * page]
            pv[p] = vc[b, :, j * page:(j + 1) * page]
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    dq = _t(q)
    got = aila_amd.gqa_decode_paged(dq, _t(pk), _t(pv), _t(table), sl, max_seq, workspace=ws)
    ref = aila_amd.gqa_decode(dq, _t(kc), _t(vc), max_seq, workspace=ws.clone(), seq_lens=sl)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    g = dg.bf16_to_f32(_np(got))
    for b, L in enumerate(lens):
        want = dg.bf16_to_f32(oracle.attention_decode_baseline(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv,
                                                               D, max_seq, L))[0]
        assert _relerr(g[b], want) <= ATTN_TOL, (b, L)


def _fused_prep_cases(sweep_seed):
    rng = np.random.default_rng(0x5EEF + sweep_seed)
    cases = []
    for i in range(10):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
        Hkv = int(rng.choice([1, 2, 4]))
        B = int(rng.integers(1, 5))
        rot = int(rng.choice([32, 64, D]))
        packed = bool(rng.integers(0, 2))
        split = bool(rng.integers(0, 2))
        max_seq = int(rng.integers(64, 2500))
        pos = [int(x) for x in rng.integers(0, max_seq, size=B)]
        cases.append((i, D, G, Hkv, B, rot, packed, split, max_seq, pos))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,B,rot,packed,split,max_seq,pos", _all(_fused_prep_cases))
def test_sweep_fused_prepare_append_decode(i, D, G, Hkv, B, rot, packed, split, max_seq, pos):
    """One launch of QK-norm + RoPE + K/V append + decode at device positions
    (decode_prepare_qkv, ElementwiseOps.cpp:105-216, then attention_decode)
    against the oracle's prep followed by its attention."""
    import torch
    import aila_amd
    Hq = Hkv * G
    seed, theta, eps = 0x5F40 + i, 1e6, 1e-6
    print(f"sweep fused prep {i}: D={D} G={G} Hkv={Hkv} B={B} rot={rot} packed={packed} split={split} "
          f"max_seq={max_seq} pos={pos}", flush=True)
    posa = np.array(pos, np.int32)
    q = dg.normal_bf16(seed, 0, (B, Hq, 2 * D if packed else D), std=2.0)
    k = dg.normal_bf16(seed, 1, (B, Hkv, D), std=2.0)
    v = dg.normal_bf16(seed, 2, (B, Hkv, D))
    qw = dg.normal_bf16(seed, 3, (D,))
    kw = dg.normal_bf16(seed, 4, (D,))
    kc = dg.normal_bf16(seed, 5, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 6, (B, Hkv, max_seq, D))
    for b, p in enumerate(pos):      # rows past the appended one are never attended
        kc[b, :, p + 1:] = 0x7FC0
        vc[b, :, p + 1:] = 0x7FC0
    kc_d, vc_d = _t(kc), _t(vc)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda") if split else None
    res = aila_amd.gqa_decode_prepare_append(
        _t(q), _t(k), _t(v), kc_d, vc_d, max_seq - 1, q_norm_w=_t(qw), k_norm_w=_t(kw), rotary_dim=rot,
        theta=theta, eps=eps, packed_gate=packed, positions=_t(posa), workspace=ws)
    torch.cuda.synchronize()
    out = res[0] if packed else res
    qo, gw, ko = oracle.decode_prepare(q, k, v, qw, kw, kc, vc, posa, B, Hq, Hkv, D, max_seq, rot, theta, eps,
                                       packed=packed)
    got = dg.bf16_to_f32(_np(out))
    assert np.isfinite(got).all()
    for b in range(B):
        want = dg.bf16_to_f32(oracle.attention_decode_baseline(qo[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv,
                                                               D, max_seq, pos[b] + 1))[0]
        assert _relerr(got[b], want) <= ATTN_TOL, f"sequence {b}"
    if packed:
        assert np.array_equal(_np(res[1]), gw)


def _layer_cases(sweep_seed):
    rng = np.random.default_rng(0x5EF1 + sweep_seed)
    cases = []
    for i in range(8):
        B = int(rng.integers(1, 4))
        Hk = int(rng.choice([1, 2, 4]))
        Hv = Hk * int(rng.choice([1, 2, 4]))
        T = int(rng.integers(1, 300))
        steps = int(rng.integers(1, 5))
        head0 = int(rng.integers(0, 3))
        wide = bool(rng.integers(0, 2))
        cases.append((i, B, Hk, Hv, T, steps, head0, wide))
    return cases


@pytest.mark.parametrize("i,B,Hk,Hv,T,steps,head0,wide", _all(_layer_cases))
def test_sweep_layer_prefill_then_decode(i, B, Hk, Hv, T, steps, head0, wide):
    """Whole DeltaNet layer (conv ring + SiLU, L2 norms, recurrence, gated
    RMSNorm; Qwen35HybridTextBackend.cpp:1640-1798): a T-token prefill, then
    decode steps, against the oracle's layer over all T + steps tokens.
    State 1e-3, outputs 1e-2, conv ring bit-exact."""
    import torch
    import aila_amd
    d = 128
    seed = 0x5F50 + i
    total = T + steps
    print(f"sweep layer {i}: B={B} Hk={Hk} Hv={Hv} T={T} steps={steps} head0={head0} wide={wide}", flush=True)
    ch = 2 * Hk * d + Hv * d
    qkv = dg.normal_bf16(seed, 0, (B, total, ch))
    z = dg.normal_bf16(seed, 1, (B, total, Hv * d))
    a = dg.normal_bf16(seed, 2, (B, total, Hv))
    b = dg.normal_bf16(seed, 3, (B, total, Hv))
    conv_w = dg.normal_bf16(seed, 4, (ch, 4), std=0.5)
    conv_state = dg.normal(seed, 5, B * 3 * ch).reshape(B, 3, ch).astype(np.float32)
    norm_w = (1.0 + dg.normal(seed, 6, d, std=0.1)).astype(np.float32)
    S0 = dg.normal(seed, 7, B * Hv * d * d, std=0.02).reshape(B, Hv, d, d).astype(np.float32)
    dtb = dg.normal_bf16(seed, 8, (Hv,))
    alog = np.log(1.0 + np.abs(dg.normal(seed, 9, Hv, std=4.0))).astype(np.float32)
    want_out, want_S, want_cs = oracle.deltanet_layer(qkv, z, a, b, conv_w, conv_state, head0, norm_w, S0, B,
                                                      total, Hk, Hv, d, d, dt_bias=dtb, A_log=alog, fast=True)
    st, cs = _t(S0), _t(conv_state)
    w, nw, dtb_d, alog_d = _t(conv_w), _t(norm_w), _t(dtb), _t(alog)
    dqkv, dz, da, db = _t(qkv), _t(z), _t(a), _t(b)
    outs = [aila_amd.deltanet_layer_prefill(dqkv[:, :T].contiguous(), dz[:, :T].contiguous(),
                                            da[:, :T].contiguous(), db[:, :T].contiguous(), w, cs, head0, nw, st,
                                            Hk, dt_bias=dtb_d, A_log=alog_d)]
    arr = torch.zeros(B * Hk, dtype=torch.int32, device="cuda") if wide else None
    for t in range(T, total):
        o = aila_amd.deltanet_layer_decode(dqkv[:, t], dz[:, t], da[:, t], db[:, t], w, cs, (head0 + t) % 3, nw,
                                           st, Hk, dt_bias=dtb_d, A_log=alog_d, arrivals=arr)
        outs.append(o.view(B, 1, Hv * d))
    torch.cuda.synchronize()
    got_out = dg.bf16_to_f32(np.concatenate([_np(o).reshape(B, -1, Hv * d) for o in outs], axis=1))
    assert _relerr(st.cpu().numpy(), want_S) <= 1e-3
    assert _relerr(got_out, dg.bf16_to_f32(want_out).reshape(B, total, Hv * d)) <= ATTN_TOL
    assert np.array_equal(cs.cpu().numpy(), want_cs)
    if wide:
        assert not arr.any()


def _append_cases(sweep_seed):
    rng = np.random.default_rng(0x5EF2 + sweep_seed)
    cases = []
    for i in range(10):
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
        Hkv = int(rng.choice([1, 2, 4]))
        B = int(rng.integers(1, 6))
        max_seq = int(rng.integers(32, 3000))
        pos = [int(x) for x in rng.integers(0, max_seq, size=B)]
        bound = int(rng.integers(max(pos), max_seq))
        cases.append((i, D, G, Hkv, B, max_seq, bound, pos))
    return cases


@pytest.mark.parametrize("i,D,G,Hkv,B,max_seq,bound,pos", _all(_append_cases))
def test_sweep_decode_append_device_positions(i, D, G, Hkv, B, max_seq, bound, pos):
    """Append + split-K decode in one launch at device positions under a host
    bound (ElementwiseOps.cpp:105-216 cache write, then
    AttentionOps.cpp:168-320): the row lands bit-exact, every sequence
    attends rows [0, pos] within tolerance, no other cache row changes."""
    import torch
    import aila_amd
    Hq = Hkv * G
    seed = 0x5F60 + i
    print(f"sweep append {i}: D={D} G={G} Hkv={Hkv} B={B} max_seq={max_seq} bound={bound} pos={pos}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kn = dg.normal_bf16(seed, 1, (B, Hkv, D))
    vn = dg.normal_bf16(seed, 2, (B, Hkv, D))
    kc = dg.normal_bf16(seed, 3, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 4, (B, Hkv, max_seq, D))
    for b, p in enumerate(pos):
        kc[b, :, p:] = 0x7FC0
        vc[b, :, p:] = 0x7FC0
    dkc, dvc = _t(kc), _t(vc)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out = aila_amd.gqa_decode_append(_t(q), _t(kn), _t(vn), dkc, dvc, bound, workspace=ws,
                                     positions=_t(np.array(pos, np.int32)))
    torch.cuda.synchronize()
    gk, gv = _np(dkc), _np(dvc)
    for b, p in enumerate(pos):
        assert np.array_equal(gk[b, :, p], kn[b]) and np.array_equal(gv[b, :, p], vn[b])
        kc[b, :, p] = kn[b]
        vc[b, :, p] = vn[b]
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)
    got = dg.bf16_to_f32(_np(out))
    for b, p in enumerate(pos):
        want = dg.bf16_to_f32(oracle.attention_decode_baseline(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv, D,
                                                               max_seq, p + 1))[0]
        assert _relerr(got[b], want) <= ATTN_TOL, (b, p)
