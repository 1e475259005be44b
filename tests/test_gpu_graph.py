"""HIP-graph replay of a decode step (fused K/V append + split-K GQA decode
with device-side positions + DeltaNet decode + position advance) matches the same
step run eagerly, replay after replay, with eager work and synchronisation
between the replays."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_graph_replay_matches_eager():
    import torch
    import aila_amd
    g = torch.Generator(device="cuda")
    g.manual_seed(123)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    B, Hq, Hkv, D, L0, max_seq = 2, 8, 2, 256, 700, 800
    Hk, Hv, d = 2, 4, 128
    kc0 = torch.randn((B, Hkv, max_seq, D), generator=g, **bf)
    vc0 = torch.randn((B, Hkv, max_seq, D), generator=g, **bf)
    st0 = torch.randn((B, Hv, d, d), generator=g, device="cuda") * 0.02
    steps = [dict(q=torch.randn((B, Hq, D), generator=g, **bf), kn=torch.randn((B, Hkv, D), generator=g, **bf),
                  vn=torch.randn((B, Hkv, D), generator=g, **bf), dq=torch.randn((B, Hk, d), generator=g, **bf),
                  dk=torch.randn((B, Hk, d), generator=g, **bf), dv=torch.randn((B, Hv, d), generator=g, **bf),
                  da=torch.randn((B, Hv), generator=g, **bf), db=torch.randn((B, Hv), generator=g, **bf))
             for _ in range(2)]
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")

    def make_state():
        return dict(kc=kc0.clone(), vc=vc0.clone(), st=st0.clone(),
                    pos=torch.full((B,), L0, dtype=torch.int32, device="cuda"),
                    lens=torch.full((B,), L0 + 1, dtype=torch.int32, device="cuda"),
                    o=torch.empty((B, Hq, D), **bf), do=torch.empty((B, Hv, d), **bf))

    def step(S, x):
        aila_amd.gqa_decode_append(x["q"], x["kn"], x["vn"], S["kc"], S["vc"], max_seq - 1, out=S["o"],
                                   workspace=ws, positions=S["pos"])
        aila_amd.deltanet_decode(x["dq"], x["dk"], x["dv"], x["da"], x["db"], S["st"], out=S["do"])
        S["pos"].add_(1)
        S["lens"].add_(1)

    eager = make_state()
    graph_s = make_state()
    graphs = []
    for x in steps:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            step(graph_s, x)
        graphs.append(gr)
    torch.cuda.synchronize()
    for i in range(6):
        x = steps[i % 2]
        step(eager, x)
        graphs[i % 2].replay()
        torch.cuda.synchronize()
        _ = (eager["o"].float().sum() + 1).item()    # unrelated eager work between replays
        assert torch.equal(graph_s["o"], eager["o"]), f"replay {i}: gqa output differs"
        assert torch.equal(graph_s["do"], eager["do"]), f"replay {i}: deltanet output differs"
        assert torch.equal(graph_s["st"], eager["st"]), f"replay {i}: state differs"
        assert torch.equal(graph_s["lens"], eager["lens"])
    assert torch.equal(graph_s["kc"], eager["kc"]) and torch.equal(graph_s["vc"], eager["vc"])
    assert int(eager["lens"][0]) == L0 + 7


def test_graph_replay_paged_decode_and_wide_layer_decode():
    """A decode step over the paged cache (paged append + paged decode with
    device lengths) and the whole DeltaNet layer with one workgroup per value
    head (self-resetting arrival counts), captured once and replayed: every
    replay equals the eager step, and the arrival counts are zero after
    each."""
    import torch
    import aila_amd
    g = torch.Generator(device="cuda")
    g.manual_seed(321)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    B, Hq, Hkv, D, page, mp, L0 = 2, 8, 2, 128, 64, 8, 300
    Hk, Hv, d = 2, 4, 128
    ch = 2 * Hk * d + Hv * d
    pk0 = torch.randn((B * mp, Hkv, page, D), generator=g, **bf)
    pv0 = torch.randn((B * mp, Hkv, page, D), generator=g, **bf)
    table = torch.randperm(B * mp, generator=torch.Generator().manual_seed(5)).to(torch.int32).view(B, mp).cuda()
    st0 = torch.randn((B, Hv, d, d), generator=g, device="cuda") * 0.02
    cs0 = torch.randn((B, 3, ch), generator=g, device="cuda")
    w = torch.randn((ch, 4), generator=g, **bf)
    nw = torch.ones(d, device="cuda")
    x = dict(q=torch.randn((B, Hq, D), generator=g, **bf), kn=torch.randn((B, Hkv, D), generator=g, **bf),
             vn=torch.randn((B, Hkv, D), generator=g, **bf), qkv=torch.randn((B, ch), generator=g, **bf),
             z=torch.randn((B, Hv * d), generator=g, **bf), a=torch.randn((B, Hv), generator=g, **bf),
             b=torch.randn((B, Hv), generator=g, **bf))
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")

    def make_state():
        return dict(pk=pk0.clone(), pv=pv0.clone(), st=st0.clone(), cs=cs0.clone(),
                    pos=torch.full((B,), L0, dtype=torch.int32, device="cuda"),
                    lens=torch.full((B,), L0 + 1, dtype=torch.int32, device="cuda"),
                    heads=torch.zeros((B,), dtype=torch.int32, device="cuda"),
                    arr=torch.zeros((B * Hk,), dtype=torch.int32, device="cuda"),
                    o=torch.empty((B, Hq, D), **bf), lo=torch.empty((B, Hv * d), **bf))

    def step(S):
        aila_amd.kv_append_paged(x["kn"], x["vn"], S["pk"], S["pv"], table, S["pos"])
        aila_amd.gqa_decode_paged(x["q"], S["pk"], S["pv"], table, S["lens"], page * mp, out=S["o"], workspace=ws)
        aila_amd.deltanet_layer_decode(x["qkv"], x["z"], x["a"], x["b"], w, S["cs"], 0, nw, S["st"], Hk,
                                       out=S["lo"], conv_heads=S["heads"], arrivals=S["arr"])
        S["pos"].add_(1)
        S["lens"].add_(1)
        S["heads"].add_(1).remainder_(3)

    eager, graph_s = make_state(), make_state()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        step(graph_s)
    torch.cuda.synchronize()
    for i in range(5):
        step(eager)
        gr.replay()
        torch.cuda.synchronize()
        _ = (eager["o"].float().sum() + 1).item()
        for key in ("o", "lo", "st", "cs", "pk", "pv", "lens", "heads"):
            assert torch.equal(graph_s[key], eager[key]), f"replay {i}: {key} differs"
        assert not graph_s["arr"].any() and not eager["arr"].any()


def test_graph_replay_prefill_cached_key_split():
    """The key-split cached prefill (partial-record pass + merge) captured
    once and replayed: every replay equals the eager call bit for bit."""
    import torch
    import aila_amd
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    S, start, Hq, Hkv, D = 96, 1900, 16, 4, 256
    max_seq = start + S
    kc = torch.randn((Hkv, max_seq, D), generator=g, **bf)
    vc = torch.randn((Hkv, max_seq, D), generator=g, **bf)
    qs = [torch.randn((S, Hq * D), generator=g, **bf) for _ in range(2)]
    need = aila_amd.gqa_prefill_cached_workspace_size(S, start, Hq, Hkv, D)
    assert need > 0
    ws_e = torch.empty(need, dtype=torch.uint8, device="cuda")
    ws_g = torch.empty(need, dtype=torch.uint8, device="cuda")
    out_e = torch.empty((S, Hq * D), **bf)
    out_g = torch.empty((S, Hq * D), **bf)
    q_in = qs[0].clone()
    aila_amd.gqa_prefill_cached(q_in, kc, vc, start, Hq, out=out_g, workspace=ws_g)   # warm the path
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        aila_amd.gqa_prefill_cached(q_in, kc, vc, start, Hq, out=out_g, workspace=ws_g)
    torch.cuda.synchronize()
    for i in range(4):
        q_in.copy_(qs[i % 2])
        aila_amd.gqa_prefill_cached(qs[i % 2], kc, vc, start, Hq, out=out_e, workspace=ws_e)
        gr.replay()
        torch.cuda.synchronize()
        _ = (out_e.float().sum() + 1).item()
        assert torch.equal(out_g, out_e), f"replay {i}"


def test_graph_replay_chunked_prefills():
    """The chunked DeltaNet prefill and the whole-layer prefill (four copies
    of the scan loop, one per slab load order) captured in one graph with
    the state reset inside it: every replay, with eager work in between,
    equals the eager call bit for bit."""
    import torch
    import aila_amd
    g = torch.Generator(device="cuda")
    g.manual_seed(321)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    B, T, Hk, Hv, d = 1, 200, 2, 4, 128
    ch = 2 * Hk * d + Hv * d
    q = torch.randn((B, T, Hk, d), generator=g, **bf)
    k = torch.randn((B, T, Hk, d), generator=g, **bf)
    v = torch.randn((B, T, Hv, d), generator=g, **bf)
    a = torch.randn((B, T, Hv), generator=g, **bf)
    b = torch.randn((B, T, Hv), generator=g, **bf)
    qkv = torch.randn((B, T, ch), generator=g, **bf)
    z = torch.randn((B, T, Hv * d), generator=g, **bf)
    conv_w = torch.randn((ch, 4), generator=g, **bf) * 0.5
    norm_w = 1.0 + 0.1 * torch.randn(d, generator=g, device="cuda")
    s0 = torch.randn((B, Hv, d, d), generator=g, device="cuda") * 0.02
    cs0 = torch.randn((B, 3, ch), generator=g, device="cuda")
    ws = torch.empty(aila_amd.deltanet_prefill_workspace_size(B, T, Hv, d, d), dtype=torch.uint8, device="cuda")
    wsl = torch.empty(aila_amd.deltanet_layer_prefill_workspace_size(B, T, Hk, Hv), dtype=torch.uint8, device="cuda")

    def make():
        return dict(st=s0.clone(), stl=s0.clone(), cs=cs0.clone(), o=torch.empty((B, T, Hv, d), **bf),
                    ol=torch.empty((B, T, Hv * d), **bf))

    def run(S):
        S["st"].copy_(s0)
        S["stl"].copy_(s0)
        S["cs"].copy_(cs0)
        aila_amd.deltanet_prefill(q, k, v, a, b, S["st"], out=S["o"], workspace=ws)
        aila_amd.deltanet_layer_prefill(qkv, z, a, b, conv_w, S["cs"], 1, norm_w, S["stl"], Hk, out=S["ol"],
                                        workspace=wsl)

    eager, graph_s = make(), make()
    run(eager)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        run(graph_s)
    for i in range(3):
        gr.replay()
        torch.cuda.synchronize()
        _ = (eager["o"].float().sum() + 1).item()   # unrelated eager work between replays
        for key in ("st", "stl", "cs", "o", "ol"):
            assert torch.equal(graph_s[key], eager[key]), f"replay {i}: {key} differs"
