"""GPU parity: the general-shape Gated DeltaNet path (the token-sequential
kernel the entry points take for shapes outside their tuned kernels: value /
key head ratios outside {1, 2, 4} or not dividing, dk or dv other than 128,
conv kernel widths other than 4). Reference role: the single-workgroup
fallback of run_linear_delta_decode_gpu (Qwen35HybridTextBackend.cpp:
1168-1304) and the token loop of run_linear_delta_prefill_gpu_batched.

Against the CPU oracle (orc_deltanet_layer / orc_deltanet_recurrent, which
follow the reference's host path including its key-head mapping for a
non-dividing head count). Tolerances: fp32 state within 1e-3 relative, bf16
outputs within 1e-2, conv ring bit-exact.
"""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg

pytestmark = pytest.mark.gpu

STATE_TOL = 1e-3
OUT_TOL = 1e-2


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


def _rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(a - r)) / max(float(np.max(np.abs(r))), 1e-30))


def _layer_inputs(seed, B, T, Hk, Hv, dk, dv, K):
    ch = 2 * Hk * dk + Hv * dv
    return dict(
        qkv=dg.normal_bf16(seed, 0, (B, T, ch)),
        z=dg.normal_bf16(seed, 1, (B, T, Hv * dv)),
        a=dg.normal_bf16(seed, 2, (B, T, Hv)),
        b=dg.normal_bf16(seed, 3, (B, T, Hv)),
        conv_w=dg.normal_bf16(seed, 4, (ch, K), std=0.5),
        conv_state=dg.normal(seed, 5, B * (K - 1) * ch).reshape(B, K - 1, ch).astype(np.float32),
        norm_w=(1.0 + dg.normal(seed, 6, dv, std=0.1)).astype(np.float32),
        state=dg.normal(seed, 7, B * Hv * dk * dv, std=0.02).reshape(B, Hv, dk, dv).astype(np.float32),
        dt_bias=dg.normal_bf16(seed, 8, (Hv,)),
        A_log=np.log(1.0 + np.abs(dg.normal(seed, 9, Hv, std=4.0))).astype(np.float32),
    )


LAYER_SHAPES = [
    # (B, Hk, Hv, dk, dv, K)
    (2, 2, 6, 128, 128, 4),    # Hv / Hk = 3
    (2, 1, 8, 128, 128, 4),    # Hv / Hk = 8
    (1, 3, 4, 128, 128, 4),    # 4 % 3 != 0: the reference's clamp mapping
    (2, 2, 4, 64, 96, 3),      # other head dims and conv width
    (1, 1, 2, 256, 256, 5),    # the largest head dims
]


@pytest.mark.parametrize("B,Hk,Hv,dk,dv,K", LAYER_SHAPES)
def test_generic_layer_decode_steps(B, Hk, Hv, dk, dv, K):
    import torch
    import aila_amd
    T, head0 = 7, 1
    x = _layer_inputs(2000 + Hv + dk, B, T, Hk, Hv, dk, dv, K)
    want_out, want_S, want_cs = oracle.deltanet_layer(
        x["qkv"], x["z"], x["a"], x["b"], x["conv_w"], x["conv_state"], head0, x["norm_w"], x["state"], B, T, Hk,
        Hv, dk, dv, K=K, dt_bias=x["dt_bias"], A_log=x["A_log"], fast=True)
    st, cs = _t(x["state"]), _t(x["conv_state"])
    w, nw, dtb, alog = _t(x["conv_w"]), _t(x["norm_w"]), _t(x["dt_bias"]), _t(x["A_log"])
    qkv, z, a, b = _t(x["qkv"]), _t(x["z"]), _t(x["a"]), _t(x["b"])
    outs = []
    for t in range(T):
        outs.append(aila_amd.deltanet_layer_decode(qkv[:, t], z[:, t], a[:, t], b[:, t], w, cs,
                                                   (head0 + t) % (K - 1), nw, st, Hk, dt_bias=dtb, A_log=alog))
    torch.cuda.synchronize()
    got = np.stack([_np(o) for o in outs], axis=1)
    assert _rel(_np(st), want_S) <= STATE_TOL
    assert _rel(dg.bf16_to_f32(got), dg.bf16_to_f32(want_out)) <= OUT_TOL
    assert np.array_equal(_np(cs), want_cs), "conv ring must hold the raw inputs bit-exact"


@pytest.mark.parametrize("B,Hk,Hv,dk,dv,K", LAYER_SHAPES[:4])
def test_generic_layer_prefill_then_decode(B, Hk, Hv, dk, dv, K):
    """Prefill over T tokens (ragged, and shorter than the ring for one case),
    then decode steps continuing the ring and the state."""
    import torch
    import aila_amd
    for T0, head0 in ((37, 2), (1, 0)):
        steps = 3
        T = T0 + steps
        x = _layer_inputs(2100 + T0 + Hv, B, T, Hk, Hv, dk, dv, K)
        want_out, want_S, want_cs = oracle.deltanet_layer(
            x["qkv"], x["z"], x["a"], x["b"], x["conv_w"], x["conv_state"], head0, x["norm_w"], x["state"], B, T,
            Hk, Hv, dk, dv, K=K, dt_bias=x["dt_bias"], A_log=x["A_log"], fast=True)
        st, cs = _t(x["state"]), _t(x["conv_state"])
        w, nw, dtb, alog = _t(x["conv_w"]), _t(x["norm_w"]), _t(x["dt_bias"]), _t(x["A_log"])
        qkv, z, a, b = _t(x["qkv"]), _t(x["z"]), _t(x["a"]), _t(x["b"])
        assert aila_amd.deltanet_layer_prefill_workspace_size(B, T0, Hk, Hv, dk, dv) == 0 or (
            dk == dv == 128 and K == 4 and Hv % Hk == 0)
        o_pre = aila_amd.deltanet_layer_prefill(qkv[:, :T0].contiguous(), z[:, :T0].contiguous(),
                                                a[:, :T0].contiguous(), b[:, :T0].contiguous(), w, cs, head0, nw,
                                                st, Hk, dt_bias=dtb, A_log=alog)
        outs = [_np(o_pre)]
        for t in range(T0, T):
            o = aila_amd.deltanet_layer_decode(qkv[:, t], z[:, t], a[:, t], b[:, t], w, cs,
                                               (head0 + t) % (K - 1), nw, st, Hk, dt_bias=dtb, A_log=alog)
            outs.append(_np(o)[:, None])
        torch.cuda.synchronize()
        got = np.concatenate(outs, axis=1)
        assert _rel(_np(st), want_S) <= STATE_TOL, f"T0={T0}"
        assert _rel(dg.bf16_to_f32(got), dg.bf16_to_f32(want_out)) <= OUT_TOL, f"T0={T0}"
        assert np.array_equal(_np(cs), want_cs), f"T0={T0}: ring"


@pytest.mark.parametrize("B,Hk,Hv,dk,dv", [(2, 3, 4, 96, 64), (3, 2, 6, 128, 128), (1, 4, 4, 32, 200)])
def test_generic_recurrence_decode_and_prefill(B, Hk, Hv, dk, dv):
    """aila_hip_deltanet_decode / _prefill on shapes outside the tuned
    kernels: a prefill over T0 tokens then decode steps, against the oracle's
    recurrence over all tokens."""
    import torch
    import aila_amd
    T0, steps = 50, 4
    T = T0 + steps
    seed = 2200 + dk + Hv
    q = dg.normal_bf16(seed, 0, (B, T, Hk, dk))
    k = dg.normal_bf16(seed, 1, (B, T, Hk, dk))
    v = dg.normal_bf16(seed, 2, (B, T, Hv, dv))
    a = dg.normal_bf16(seed, 3, (B, T, Hv))
    b = dg.normal_bf16(seed, 4, (B, T, Hv))
    S0 = dg.normal(seed, 5, B * Hv * dk * dv, std=0.02).reshape(B, Hv, dk, dv).astype(np.float32)
    _, want_o, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T, Hk, Hv, dk, dv)
    st = _t(S0)
    o_pre = aila_amd.deltanet_prefill(_t(q[:, :T0]), _t(k[:, :T0]), _t(v[:, :T0]), _t(a[:, :T0]),
                                      _t(b[:, :T0]), st)
    outs = [_np(o_pre)]
    for t in range(T0, T):
        o = aila_amd.deltanet_decode(_t(q[:, t]), _t(k[:, t]), _t(v[:, t]), _t(a[:, t]), _t(b[:, t]), st)
        outs.append(_np(o)[:, None])
    torch.cuda.synchronize()
    got = np.concatenate(outs, axis=1)
    assert _rel(_np(st), want_S) <= STATE_TOL
    assert _rel(dg.bf16_to_f32(got), dg.bf16_to_f32(want_o)) <= OUT_TOL


def test_generic_prefill_2048_tokens_state():
    """2048 sequential tokens on the general path (6 value heads over 4 key
    heads: the clamp mapping, no tuned kernel): the state
    stays within 1e-3 of the fp32 oracle, with slow decays (long memory)."""
    import torch
    import aila_amd
    B, Hk, Hv, dk, dv, T = 1, 4, 6, 128, 128, 2048
    seed = 2300
    q = dg.normal_bf16(seed, 0, (B, T, Hk, dk))
    k = dg.normal_bf16(seed, 1, (B, T, Hk, dk))
    v = dg.normal_bf16(seed, 2, (B, T, Hv, dv))
    a = dg.f32_to_bf16(np.full((B, T, Hv), -6.0, np.float32))    # decay ~ e^-0.0025
    b = dg.normal_bf16(seed, 4, (B, T, Hv))
    S0 = dg.normal(seed, 5, B * Hv * dk * dv, std=0.02).reshape(B, Hv, dk, dv).astype(np.float32)
    _, want_o, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T, Hk, Hv, dk, dv)
    st = _t(S0)
    o = aila_amd.deltanet_prefill(_t(q), _t(k), _t(v), _t(a), _t(b), st)
    torch.cuda.synchronize()
    assert _rel(_np(st), want_S) <= STATE_TOL
    assert _rel(dg.bf16_to_f32(_np(o)), dg.bf16_to_f32(want_o)) <= OUT_TOL
