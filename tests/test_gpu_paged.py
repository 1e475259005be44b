"""GPU parity of the paged-KV decode (aila_hip_gqa_decode_paged) and the
paged append (aila_hip_kv_append_paged).

The same cache rows are laid out contiguously ([B, Hkv, max_seq, D], the
reference's per-sequence [Hkv, max_seq, D] cache, KVCache.hpp:9-45) and
scattered over a shuffled page pool; the paged decode must equal the
contiguous decode bit for bit (same split plan, same rows) and the CPU
oracle (AttentionOps.cpp:73-166) within the attention tolerance (max
relative error 1e-2). Pool pages no sequence owns hold NaN, so any read of a
wrong page poisons the output.
"""
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


def _paged_layout(seed, kc, vc, page_size, spare=5):
    """Scatter [B, Hkv, max_seq, D] into a shuffled pool [P, Hkv, page_size, D]
    (+ spare NaN pages); returns pool_k, pool_v, table [B, max_pages]."""
    B, Hkv, max_seq, D = kc.shape
    mp = max_seq // page_size
    npages = B * mp + spare
    rng = np.random.default_rng(seed)
    perm = rng.permutation(npages)
    pool_k = np.full((npages, Hkv, page_size, D), 0x7FC0, np.uint16)
    pool_v = np.full((npages, Hkv, page_size, D), 0x7FC0, np.uint16)
    table = np.zeros((B, mp), np.int32)
    for b in range(B):
        for j in range(mp):
            p = int(perm[b * mp + j])
            table[b, j] = p
            pool_k[p] = kc[b, :, j * page_size:(j + 1) * page_size]
            pool_v[p] = vc[b, :, j * page_size:(j + 1) * page_size]
    return pool_k, pool_v, table


@pytest.mark.parametrize("page_size,D,G", [(16, 256, 4), (64, 128, 2), (256, 256, 4), (128, 64, 8)])
def test_paged_decode_matches_contiguous_and_oracle(page_size, D, G):
    import torch
    import aila_amd
    B, Hkv, max_seq = 3, 2, 2048
    Hq = Hkv * G
    lens = [2048, 1000, 1] if page_size != 64 else [960, 1008, 100]
    seed = 0x9A6E + page_size + D
    print(f"paged decode page_size={page_size} D={D} G={G} lens={lens}", flush=True)
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    for b, L in enumerate(lens):      # rows past each length are never attended
        kc[b, :, L:] = 0x7FC0
        vc[b, :, L:] = 0x7FC0
    pk, pv, table = _paged_layout(seed, kc, vc, page_size)
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    dq = _t(q)
    for workspace in (ws, None):
        got = aila_amd.gqa_decode_paged(dq, _t(pk), _t(pv), _t(table), sl, max_seq, workspace=workspace)
        ref = aila_amd.gqa_decode(dq, _t(kc), _t(vc), max_seq, workspace=workspace, seq_lens=sl)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), "paged and contiguous decode differ"
        g = dg.bf16_to_f32(_np(got))
        assert np.isfinite(g).all()
        for b, L in enumerate(lens):
            want = dg.bf16_to_f32(oracle.attention_decode_baseline(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq,
                                                                   Hkv, D, max_seq, L))[0]
            assert _relerr(g[b], want) <= ATTN_TOL, (b, L)


def test_paged_append_then_decode():
    import torch
    import aila_amd
    B, Hkv, Hq, D, max_seq, page_size = 2, 4, 16, 256, 1024, 64
    seed = 0x9A70
    q = dg.normal_bf16(seed, 0, (B, Hq, D))
    kc = dg.normal_bf16(seed, 1, (B, Hkv, max_seq, D))
    vc = dg.normal_bf16(seed, 2, (B, Hkv, max_seq, D))
    kn = dg.normal_bf16(seed, 3, (B, Hkv, D))
    vn = dg.normal_bf16(seed, 4, (B, Hkv, D))
    pos = [700, 63]
    for b, p in enumerate(pos):
        kc[b, :, p:] = 0x7FC0
        vc[b, :, p:] = 0x7FC0
    pk, pv, table = _paged_layout(seed, kc, vc, page_size)
    dpk, dpv, dtab = _t(pk), _t(pv), _t(table)
    dpos = torch.tensor(pos, dtype=torch.int32, device="cuda")
    aila_amd.kv_append_paged(_t(kn), _t(vn), dpk, dpv, dtab, dpos)
    lens = torch.tensor([p + 1 for p in pos], dtype=torch.int32, device="cuda")
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out = aila_amd.gqa_decode_paged(_t(q), dpk, dpv, dtab, lens, max_seq, workspace=ws)
    torch.cuda.synchronize()
    gk, gv = _np(dpk), _np(dpv)
    for b, p in enumerate(pos):
        page = table[b, p // page_size]
        assert np.array_equal(gk[page, :, p % page_size], kn[b]) and np.array_equal(gv[page, :, p % page_size], vn[b])
        kc[b, :, p] = kn[b]
        vc[b, :, p] = vn[b]
    # nothing else in the pool changed
    for b, p in enumerate(pos):
        page = table[b, p // page_size]
        gk[page, :, p % page_size] = pk[page, :, p % page_size]
        gv[page, :, p % page_size] = pv[page, :, p % page_size]
    assert np.array_equal(gk, pk) and np.array_equal(gv, pv)
    g = dg.bf16_to_f32(_np(out))
    for b, p in enumerate(pos):
        want = dg.bf16_to_f32(oracle.attention_decode_baseline(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], 1, Hq, Hkv, D,
                                                               max_seq, p + 1))[0]
        assert _relerr(g[b], want) <= ATTN_TOL


def test_paged_rejects_bad_arguments():
    import torch
    import aila_amd
    q = torch.zeros((1, 8, 128), dtype=torch.bfloat16, device="cuda")
    pages = torch.zeros((4, 2, 24, 128), dtype=torch.bfloat16, device="cuda")
    table = torch.zeros((1, 4), dtype=torch.int32, device="cuda")
    sl = torch.ones((1,), dtype=torch.int32, device="cuda")
    with pytest.raises(aila_amd.AilaHipError):
        aila_amd.gqa_decode_paged(q, pages, pages, table, sl, 10)          # page_size 24 not a multiple of 16
    pages = torch.zeros((4, 2, 32, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(aila_amd.AilaHipError):
        aila_amd.gqa_decode_paged(q, pages, pages, table, sl, 4 * 32 + 1)  # max_len beyond the table
