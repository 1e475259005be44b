"""Committed golden vectors (tests/golden/fixtures.npz, written by
tests/golden/make_fixtures.py from the CPU oracle and the seeded generator).

CPU: the oracle and the generator reproduce every committed array bit for
bit, so a change to either that moves a result shows up here.
GPU: the HIP path against the committed outputs, at the path's tolerances
(bf16 outputs: max |a - r| / max |r| <= 1e-2; fp32 state: the same ratio
<= 1e-3 on the committed sample and summary; the conv ring, raw inputs,
bit-exact).
"""
import importlib.util
import os

import numpy as np
import pytest

from aila_amd import datagen as dg

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("make_fixtures", os.path.join(HERE, "golden", "make_fixtures.py"))
mf = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mf)

OUT_TOL = 1e-2
STATE_TOL = 1e-3


def _fixture():
    with np.load(os.path.join(HERE, "golden", "fixtures.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(a - r)) / max(float(np.max(np.abs(r))), 1e-30))


def test_oracle_reproduces_fixtures():
    want = _fixture()
    got = mf.compute()
    assert sorted(got) == sorted(want)
    for k in want:
        assert got[k].dtype == want[k].dtype and got[k].shape == want[k].shape, k
        assert np.array_equal(got[k].view(np.uint8), want[k].view(np.uint8)), f"{k} differs from the fixture"


def test_fixture_outputs_are_finite_and_nontrivial():
    f = _fixture()
    for k, v in f.items():
        if k.endswith("/out"):
            x = dg.bf16_to_f32(v)
            assert np.isfinite(x).all() and np.abs(x).max() > 0, k


# ---------------------------------------------------------------- GPU ----
def _t(x):
    import torch
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _np(t):
    import torch
    if t.dtype == torch.bfloat16:
        return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)
    return t.detach().cpu().numpy()


def _check_state(name, st, f):
    stats, sample = mf.state_summary(st)
    assert _rel(sample, f[f"{name}/state_sample"]) <= STATE_TOL, "state sample"
    assert abs(stats[1] - f[f"{name}/state_stats"][1]) <= STATE_TOL * f[f"{name}/state_stats"][1], "state max"
    assert abs(stats[0] - f[f"{name}/state_stats"][0]) <= STATE_TOL * np.abs(st).sum(), "state sum"


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["decode128", "decode256"])
def test_gpu_decode_matches_fixture(name):
    import torch
    import aila_amd
    f, c = _fixture(), mf.CASES[name]
    q, kc, vc = mf.decode_inputs(c["seed"], c["B"], c["Hq"], c["Hkv"], c["D"], c["L"])
    assert np.array_equal(mf.checksum(q, kc, vc), f[f"{name}/inputs"])
    for split in (False, True):
        ws = None
        if split:
            ws = torch.empty(aila_amd.gqa_decode_workspace_size(c["B"], c["Hq"], c["D"]), dtype=torch.uint8,
                             device="cuda")
        print(f"golden {name} split={split}", flush=True)
        out = aila_amd.gqa_decode(_t(q), _t(kc), _t(vc), c["L"], workspace=ws)
        torch.cuda.synchronize()
        assert _rel(dg.bf16_to_f32(_np(out)), dg.bf16_to_f32(f[f"{name}/out"])) <= OUT_TOL


@pytest.mark.gpu
def test_gpu_prefill_matches_fixture():
    import torch
    import aila_amd
    f, c = _fixture(), mf.CASES["prefill64"]
    q, k, v = mf.prefill_inputs(c["seed"], c["S"], c["Hq"], c["Hkv"], c["D"])
    out = aila_amd.gqa_prefill(_t(q), _t(k), _t(v), c["Hq"], c["Hkv"])
    torch.cuda.synchronize()
    assert _rel(dg.bf16_to_f32(_np(out)), dg.bf16_to_f32(f["prefill64/out"])) <= OUT_TOL


@pytest.mark.gpu
def test_gpu_prefill_cached_matches_fixture():
    import torch
    import aila_amd
    f, c = _fixture(), mf.CASES["cached128"]
    q, kc, vc = mf.cached_inputs(c["seed"], c["S"], c["start"], c["Hq"], c["Hkv"], c["D"], c["max_seq"])
    out = aila_amd.gqa_prefill_cached(_t(q), _t(kc), _t(vc), c["start"], c["Hq"])
    torch.cuda.synchronize()
    assert _rel(dg.bf16_to_f32(_np(out)), dg.bf16_to_f32(f["cached128/out"])) <= OUT_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("chunked", [False, True])
def test_gpu_deltanet_matches_fixture(chunked):
    import torch
    import aila_amd
    f, c = _fixture(), mf.CASES["deltanet"]
    x = mf.deltanet_inputs(c["seed"], c["B"], c["T"], c["Hk"], c["Hv"], c["d"])
    st = _t(x["state"])
    q, k, v, a, b = (_t(x[n]) for n in ("q", "k", "v", "a", "b"))
    if chunked:
        out = _np(aila_amd.deltanet_prefill(q, k, v, a, b, st))
    else:
        out = np.stack([_np(aila_amd.deltanet_decode(q[:, t], k[:, t], v[:, t], a[:, t], b[:, t], st))
                        for t in range(c["T"])], axis=1)
    torch.cuda.synchronize()
    assert _rel(dg.bf16_to_f32(out), dg.bf16_to_f32(f["deltanet/out"])) <= OUT_TOL
    _check_state("deltanet", _np(st), f)


@pytest.mark.gpu
@pytest.mark.parametrize("prefill", [False, True])
def test_gpu_deltanet_layer_matches_fixture(prefill):
    import torch
    import aila_amd
    f, c = _fixture(), mf.CASES["layer"]
    x = mf.layer_inputs(c["seed"], c["B"], c["T"], c["Hk"], c["Hv"], c["d"])
    st, cs = _t(x["state"]), _t(x["conv_state"])
    w, nw, dtb, alog = _t(x["conv_w"]), _t(x["norm_w"]), _t(x["dt_bias"]), _t(x["A_log"])
    qkv, z, a, b = _t(x["qkv"]), _t(x["z"]), _t(x["a"]), _t(x["b"])
    if prefill:
        out = _np(aila_amd.deltanet_layer_prefill(qkv, z, a, b, w, cs, c["head"], nw, st, c["Hk"], dt_bias=dtb,
                                                  A_log=alog))
    else:
        out = np.stack([_np(aila_amd.deltanet_layer_decode(qkv[:, t], z[:, t], a[:, t], b[:, t], w, cs,
                                                           (c["head"] + t) % 3, nw, st, c["Hk"], dt_bias=dtb,
                                                           A_log=alog)) for t in range(c["T"])], axis=1)
    torch.cuda.synchronize()
    assert _rel(dg.bf16_to_f32(out), dg.bf16_to_f32(f["layer/out"])) <= OUT_TOL
    _check_state("layer", _np(st), f)
    assert np.array_equal(_np(cs), f["layer/conv_state"]), "conv ring holds the raw inputs bit-exact"
