"""GPU parity: chunked Gated DeltaNet prefill vs the sequential fp32 oracle
recurrence (run_linear_delta_host, Qwen35HybridTextBackend.cpp:1729-1780).

Tolerances: bf16 outputs within max relative error 1e-2; the fp32 final
state within 1e-3 relative (max-norm).
"""
import numpy as np
import pytest

import oracle
from aila_amd import datagen as dg

pytestmark = pytest.mark.gpu
OUT_TOL = 1e-2
STATE_TOL = 1e-3


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


def _case(seed, B, T, Hk, Hv, d=128, s0_std=0.02, gates=False):
    import torch
    import aila_amd
    q = dg.normal_bf16(seed, 0, (B, T, Hk, d))
    k = dg.normal_bf16(seed, 1, (B, T, Hk, d))
    v = dg.normal_bf16(seed, 2, (B, T, Hv, d))
    a = dg.normal_bf16(seed, 3, (B, T, Hv))
    b = dg.normal_bf16(seed, 4, (B, T, Hv))
    S0 = (dg.normal(seed, 5, B * Hv * d * d, std=s0_std).reshape(B, Hv, d, d)
          if s0_std > 0 else np.zeros((B, Hv, d, d), np.float32))
    dtb = dg.normal_bf16(seed, 6, (Hv,), std=0.5) if gates else None
    alog = dg.normal(seed, 7, Hv, std=0.3) if gates else None
    st = _t(S0.astype(np.float32))
    out = aila_amd.deltanet_prefill(_t(q), _t(k), _t(v), _t(a), _t(b), st,
                                    dt_bias=_t(dtb) if gates else None,
                                    A_log=_t(alog) if gates else None)
    torch.cuda.synchronize()
    _, want_ob, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T, Hk, Hv, d, d,
                                                   dt_bias=dtb, A_log=alog)
    got_o = dg.bf16_to_f32(_np(out))
    got_S = st.cpu().numpy()
    assert np.isfinite(got_o).all() and np.isfinite(got_S).all()
    eo = _relerr(got_o, dg.bf16_to_f32(want_ob))
    es = _relerr(got_S, want_S)
    assert eo <= OUT_TOL, f"out relerr {eo}"
    assert es <= STATE_TOL, f"state relerr {es}"
    return eo, es


def test_prefill_config4_qwen35():
    # benchmark config 4: T=4096, chunk 64, 16 q/k heads, 32 v heads, zero state.
    _case(0xA11A + 3, 1, 4096, 16, 32, s0_std=0.0)


def test_prefill_long_sequence():
    # 32k tokens (512 chunks) through one head pair: the state is carried
    # across the whole chain within 1e-3, outputs within 1e-2.
    print("deltanet prefill T=32768 Hk=1 Hv=2", flush=True)
    _case(0xA11A + 40, 1, 32768, 1, 2, gates=True)


@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 130, 200])
def test_prefill_ragged_lengths(T):
    _case(8000 + T, 2, T, 2, 4, gates=True)


def test_prefill_shared_key_heads_and_gates():
    _case(8100, 1, 512, 1, 4, gates=True)


def test_prefill_then_decode_continues_the_state():
    import torch
    import aila_amd
    B, T, H, d = 1, 100, 2, 128
    q = dg.normal_bf16(8200, 0, (B, T + 3, H, d))
    k = dg.normal_bf16(8200, 1, (B, T + 3, H, d))
    v = dg.normal_bf16(8200, 2, (B, T + 3, H, d))
    a = dg.normal_bf16(8200, 3, (B, T + 3, H))
    b = dg.normal_bf16(8200, 4, (B, T + 3, H))
    S0 = np.zeros((B, H, d, d), np.float32)
    st = _t(S0)
    aila_amd.deltanet_prefill(_t(q[:, :T]), _t(k[:, :T]), _t(v[:, :T]), _t(a[:, :T]), _t(b[:, :T]), st)
    outs = []
    for t in range(T, T + 3):
        outs.append(aila_amd.deltanet_decode(_t(q[:, t]), _t(k[:, t]), _t(v[:, t]), _t(a[:, t]),
                                             _t(b[:, t]), st))
    torch.cuda.synchronize()
    _, want_ob, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T + 3, H, H, d, d)
    assert _relerr(st.cpu().numpy(), want_S) <= STATE_TOL
    got = dg.bf16_to_f32(_np(torch.stack(outs, 1)))
    assert _relerr(got, dg.bf16_to_f32(want_ob[:, T:])) <= OUT_TOL


def test_prefill_rejects_bad_args():
    import torch
    import aila_amd
    # dk = 64 runs the general-shape kernel; head dims above 256 run nowhere
    q = torch.zeros((1, 8, 2, 320), dtype=torch.bfloat16, device="cuda")
    v = torch.zeros((1, 8, 2, 64), dtype=torch.bfloat16, device="cuda")
    ab = torch.zeros((1, 8, 2), dtype=torch.bfloat16, device="cuda")
    st = torch.zeros((1, 2, 320, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(aila_amd.AilaHipError):
        aila_amd.deltanet_prefill(q, q, v, ab, ab, st)


@pytest.mark.parametrize("decay", [0.9, 0.99, 0.999])
def test_prefill_slow_decays_keep_state_accuracy(decay):
    """Decays near 1 (long-memory heads): the chunk's W S nearly cancels U,
    so the state error is most sensitive to operand rounding here. A_log is
    set so that exp(-softplus(a + dt_bias) * exp(A_log)) ~ decay at a = 0."""
    import torch
    import aila_amd
    B, T, H, d = 1, 2048, 4, 128
    dtb_v = -4.0
    alog = np.full(H, np.log(-np.log(decay) / np.log1p(np.exp(dtb_v))), np.float32)
    dtb = dg.f32_to_bf16(np.full(H, dtb_v, np.float32))
    q = dg.normal_bf16(801, 0, (B, T, H, d))
    k = dg.normal_bf16(801, 1, (B, T, H, d))
    v = dg.normal_bf16(801, 2, (B, T, H, d))
    a = dg.normal_bf16(801, 3, (B, T, H), std=0.3)
    b = dg.normal_bf16(801, 4, (B, T, H))
    S0 = np.zeros((B, H, d, d), np.float32)
    st = _t(S0)
    out = aila_amd.deltanet_prefill(_t(q), _t(k), _t(v), _t(a), _t(b), st, dt_bias=_t(dtb), A_log=_t(alog))
    torch.cuda.synchronize()
    _, want_ob, want_S = oracle.deltanet_recurrent(q, k, v, a, b, S0, B, T, H, H, d, d, dt_bias=dtb, A_log=alog,
                                                   fast=True)
    es = _relerr(st.cpu().numpy(), want_S)
    eo = _relerr(dg.bf16_to_f32(_np(out)), dg.bf16_to_f32(want_ob))
    assert es <= STATE_TOL, f"state relerr {es}"
    assert eo <= OUT_TOL, f"out relerr {eo}"
