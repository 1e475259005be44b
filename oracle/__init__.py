"""ctypes bindings for the CPU oracle (``oracle/oracle.cpp``).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()``
(as the checker) and ``bench.py``'s cpu_baseline leg. The product package
``aila_amd`` never imports this module.

All array arguments are numpy arrays; bf16 tensors are ``uint16`` bit
patterns. Functions allocate and return their outputs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict = {}

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64

_SIGS = {
    "orc_f32_to_bf16_array": [_P, _P, _I64],
    "orc_bf16_to_f32_array": [_P, _P, _I64],
    "orc_num_threads": [],
    "orc_set_num_threads": [_I],
    "orc_attention_decode_baseline": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I],
    "orc_attention_decode_window": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I],
    "orc_attention_decode_splitk": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    "orc_attention_prefill_naive": [_P, _P, _P, _P, _I, _I, _I, _I],
    "orc_attention_prefill_online": [_P, _P, _P, _P, _I, _I, _I, _I, _I],
    "orc_attention_prefill_cached": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I],
    "orc_copy_to_cache": [_P, _P, _I, _I, _I, _I, _I],
    "orc_attention_f64": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I],
    "orc_head_rms_norm": [_P, _P, _P, _F, _I, _I, _I],
    "orc_apply_rope": [_P, _P, _I, _I, _I, _I, _I, _I, _F],
    "orc_decode_prepare_qkv_freq": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I],
    "orc_apply_rope_partial": [_P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _I, _I, _I, _I, _I],
    "orc_decode_prepare_rp": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                              _I, _I, _I, _I, _I, _I, _F, _F, _P,
                              _I, _P, _P, _P, _I, _I, _I, _P, _P, _I, _I, _I],
    "orc_decode_prepare_qkv": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _I],
    "orc_decode_prepare": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                           _I, _I, _I, _I, _I, _I, _F, _F, _P],
    "orc_sigmoid_mul": [_P, _P, _P, ctypes.c_long],
    "orc_deltanet_recurrent": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _I, _I, _I, _I, _I, _I, _F, _F, _I],
    "orc_deltanet_recurrent_f64": [_P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _I, _I, _I, _I, _I, _I, _F, _F, _I],
    "orc_deltanet_layer": [_P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _P, _P, _P,
                           _I, _I, _I, _I, _I, _I, _I, _F, _F],
}


def build(force: bool = False) -> None:
    """Compile liboracle.so / liboracle_fast.so with the committed Makefile."""
    args = ["make", "-C", _HERE]
    if force:
        args.append("-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)


def lib(fast: bool = False) -> ctypes.CDLL:
    name = "liboracle_fast.so" if fast else "liboracle.so"
    if name not in _LIBS:
        path = os.path.join(_HERE, name)
        if not os.path.exists(path):
            build()
        l = ctypes.CDLL(path)
        for fn, argt in _SIGS.items():
            if hasattr(l, fn):
                f = getattr(l, fn)
                f.argtypes = argt
                f.restype = _I if fn == "orc_num_threads" else None
        _LIBS[name] = l
    return _LIBS[name]


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


U16 = np.uint16
F32 = np.float32


def attention_decode_baseline(q, kc, vc, B, Hq, Hkv, D, max_seq, L, fast=False):
    q, kc, vc = _c(q, U16), _c(kc, U16), _c(vc, U16)
    out = np.zeros((B, Hq, D), U16)
    lib(fast).orc_attention_decode_baseline(_p(q), _p(kc), _p(vc), _p(out), B, Hq, Hkv, D, max_seq, L)
    return out


def attention_decode_window(q, kc, vc, B, Hq, Hkv, D, max_seq, L, window, window_start, sink, lens=None):
    """ops::attention_decode with the decode window / sink knobs; per-sequence
    lengths ``lens`` (int [B]) or L for all."""
    q, kc, vc = _c(q, U16), _c(kc, U16), _c(vc, U16)
    lens = None if lens is None else np.ascontiguousarray(lens, dtype=np.int32)
    out = np.zeros((B, Hq, D), U16)
    lib().orc_attention_decode_window(_p(q), _p(kc), _p(vc), _p(out), B, Hq, Hkv, D, max_seq, L, _p(lens),
                                      int(window), int(window_start), int(sink))
    return out


def attention_decode_splitk(q, kc, vc, B, Hq, Hkv, D, max_seq, L, tile=128,
                            want_partials=False, fast=False):
    q, kc, vc = _c(q, U16), _c(kc, U16), _c(vc, U16)
    out = np.zeros((B, Hq, D), U16)
    nt = (L + tile - 1) // tile
    part = np.zeros((B, Hq, nt, 16 + D), F32) if want_partials else None
    lib(fast).orc_attention_decode_splitk(_p(q), _p(kc), _p(vc), _p(out), B, Hq, Hkv, D,
                                          max_seq, L, tile, _p(part))
    return (out, part) if want_partials else out


def attention_prefill_naive(q, k, v, S, Hq, Hkv, D, fast=False):
    q, k, v = _c(q, U16), _c(k, U16), _c(v, U16)
    out = np.zeros((S, Hq * D), U16)
    lib(fast).orc_attention_prefill_naive(_p(q), _p(k), _p(v), _p(out), S, Hq, Hkv, D)
    return out


def attention_prefill_online(q, k, v, S, Hq, Hkv, D, tile=128, fast=False):
    q, k, v = _c(q, U16), _c(k, U16), _c(v, U16)
    out = np.zeros((S, Hq * D), U16)
    lib(fast).orc_attention_prefill_online(_p(q), _p(k), _p(v), _p(out), S, Hq, Hkv, D, tile)
    return out


def attention_prefill_cached(q, kc, vc, S, start_pos, Hq, Hkv, D, max_seq, online=False, fast=False):
    q, kc, vc = _c(q, U16), _c(kc, U16), _c(vc, U16)
    out = np.zeros((S, Hq * D), U16)
    lib(fast).orc_attention_prefill_cached(_p(q), _p(kc), _p(vc), _p(out), S, start_pos, Hq,
                                           Hkv, D, max_seq, int(online))
    return out


def copy_to_cache(src, cache, S, start_pos, H, D, max_seq):
    src = _c(src, U16)
    assert cache.dtype == U16 and cache.flags.c_contiguous
    lib().orc_copy_to_cache(_p(src), _p(cache), S, start_pos, H, D, max_seq)
    return cache


def attention_f64(q, kc, vc, S, start_pos, Hq, Hkv, D, max_seq):
    q, kc, vc = _c(q, U16), _c(kc, U16), _c(vc, U16)
    out = np.zeros((S, Hq, D), np.float64)
    lib().orc_attention_f64(_p(q), _p(kc), _p(vc), _p(out), S, start_pos, Hq, Hkv, D, max_seq)
    return out


def head_rms_norm(x, eps, S, H, D, w_bf16=None, w_f32=None):
    x = np.array(x, dtype=U16, copy=True, order="C")
    w_bf16, w_f32 = _c(w_bf16, U16), _c(w_f32, F32)
    lib().orc_head_rms_norm(_p(x), _p(w_bf16), _p(w_f32), eps, S, H, D)
    return x


def _rope_fields(rope):
    """Unpack a rotary-position dict: interleaved, pos_t/pos_h/pos_w (int
    arrays [P] or [B, P]), prompt_pos_len, text_pos_delta, prompt_lens and
    deltas (int [B]), sections (t, h, w)."""
    rope = rope or {}
    streams = [rope.get(n) for n in ("pos_t", "pos_h", "pos_w")]
    streams = [None if a is None else np.ascontiguousarray(a, dtype=np.int32) for a in streams]
    stride = 0
    if streams[0] is not None and streams[0].ndim == 2:
        stride = streams[0].shape[1]
    pl, dl = rope.get("prompt_lens"), rope.get("deltas")
    pl = None if pl is None else np.ascontiguousarray(pl, dtype=np.int32)
    dl = None if dl is None else np.ascontiguousarray(dl, dtype=np.int32)
    sec = tuple(int(x) for x in rope.get("sections", (0, 0, 0)))
    return (int(bool(rope.get("interleaved", True))), streams, stride, int(rope.get("prompt_pos_len", 0)),
            int(rope.get("text_pos_delta", 0)), pl, dl, sec)


def apply_rope(q, k, S, start_pos, Hq, Hkv, D, rotary_dim, theta, rope=None):
    """apply_rope_partial; ``rope`` (dict, see _rope_fields) gives the text
    shift and mRoPE streams (one sequence: streams [P])."""
    q = np.array(q, dtype=U16, copy=True, order="C")
    k = np.array(k, dtype=U16, copy=True, order="C")
    if rope is None:
        lib().orc_apply_rope(_p(q), _p(k), S, start_pos, Hq, Hkv, D, rotary_dim, theta)
        return q, k
    il, (pt, ph, pw), _, plen, delta, _, _, sec = _rope_fields(rope)
    lib().orc_apply_rope_partial(_p(q), _p(k), S, start_pos, Hq, Hkv, D, rotary_dim, theta, il, _p(pt), _p(ph),
                                 _p(pw), plen, delta, *sec)
    return q, k


def decode_prepare_qkv(q, k, v, qn_w, kn_w, kc, vc, start_pos, Hq, Hkv, D, eps, theta, max_seq):
    q = np.array(q, dtype=U16, copy=True, order="C")
    k = np.array(k, dtype=U16, copy=True, order="C")
    v, qn_w, kn_w = _c(v, U16), _c(qn_w, U16), _c(kn_w, U16)
    assert kc.dtype == U16 and vc.dtype == U16
    lib().orc_decode_prepare_qkv(_p(q), _p(k), _p(v), _p(qn_w), _p(kn_w), _p(kc), _p(vc),
                                 start_pos, Hq, Hkv, D, eps, theta, max_seq)
    return q, k


def decode_prepare_qkv_freq(q, k, v, rope_freq, qn_w, kn_w, kc, vc, start_pos, Hq, Hkv, D, eps, max_seq):
    """decode_prepare_qkv with the backend's rope_freq table (one sequence);
    returns (q, k); kc/vc (uint16 arrays or None) are updated."""
    q = np.array(q, dtype=U16, copy=True, order="C")
    k = np.array(k, dtype=U16, copy=True, order="C")
    v, qn_w, kn_w = _c(v, U16), _c(qn_w, U16), _c(kn_w, U16)
    f = np.ascontiguousarray(rope_freq, dtype=F32)
    lib().orc_decode_prepare_qkv_freq(_p(q), _p(k), _p(v), _p(f), _p(qn_w), _p(kn_w), _p(kc), _p(vc),
                                      start_pos, Hq, Hkv, D, eps, max_seq)
    return q, k


def decode_prepare(q_in, k, v, qn_w, kn_w, kc, vc, pos, B, Hq, Hkv, D, max_seq, rotary_dim,
                   theta, eps, packed=False, rope=None):
    """Batched decode_prepare_qkv(_partial / qgkv_packed). Returns
    (q_out, gate_out or None, k); kc/vc (uint16 arrays or None) are updated.
    ``rope``: rotary positions as in apply_rope (streams [P] shared or
    [B, P] per sequence; prompt_lens/deltas per sequence)."""
    q_in = _c(q_in, U16)
    k = np.array(k, dtype=U16, copy=True, order="C")
    v, qn_w, kn_w = _c(v, U16), _c(qn_w, U16), _c(kn_w, U16)
    q_out = np.zeros((B, Hq, D), U16)
    gate = np.zeros((B, Hq, D), U16) if packed else None
    posa = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (B,)))
    if kc is not None:
        assert kc.dtype == U16 and vc.dtype == U16 and kc.flags.c_contiguous
    il, (pt, ph, pw), stride, plen, delta, pl, dl, sec = _rope_fields(rope)
    lib().orc_decode_prepare_rp(_p(q_in), int(bool(packed)), _p(q_out), _p(gate), _p(k), _p(v), _p(qn_w),
                                _p(kn_w), _p(kc), _p(vc), B, Hq, Hkv, D, max_seq, rotary_dim, theta, eps,
                                _p(posa), il if rope else 0, _p(pt), _p(ph), _p(pw), stride, plen, delta,
                                _p(pl), _p(dl), *sec)
    return q_out, gate, k


def sigmoid_mul(x, g):
    x, g = _c(x, U16), _c(g, U16)
    o = np.zeros_like(x)
    lib().orc_sigmoid_mul(_p(x), _p(g), _p(o), x.size)
    return o


def deltanet_recurrent(q, k, v, a, b, state, B, T, Hk, Hv, dk, dv, eps=1e-6,
                       scale=None, l2norm=True, dt_bias=None, A_log=None, fast=False):
    """Returns (out_f32 [B,T,Hv,dv], out_bf16, state_after) ; state is copied."""
    if scale is None:
        scale = 1.0 / np.sqrt(dk)
    q, k, v, a, b = (_c(x, U16) for x in (q, k, v, a, b))
    dt_bias, A_log = _c(dt_bias, U16), _c(A_log, F32)
    st = np.array(state, dtype=F32, copy=True, order="C")
    out = np.zeros((B, T, Hv, dv), F32)
    outb = np.zeros((B, T, Hv, dv), U16)
    lib(fast).orc_deltanet_recurrent(_p(q), _p(k), _p(v), _p(a), _p(b), _p(dt_bias), _p(A_log),
                                     _p(st), _p(out), _p(outb), B, T, Hk, Hv, dk, dv, eps, scale,
                                     int(l2norm))
    return out, outb, st


def deltanet_layer(qkv, z, a, b, conv_w, conv_state, conv_head, norm_w, state, B, T, Hk, Hv, dk, dv,
                   K=4, eps=1e-6, scale=None, dt_bias=None, A_log=None, fast=False):
    """Full layer: conv1d ring + SiLU, L2 norm, recurrence, gated RMSNorm.
    qkv [B,T,2*Hk*dk+Hv*dv], z [B,T,Hv*dv], a/b [B,T,Hv] (uint16 bf16),
    conv_w [ch,K] bf16, conv_state [B,K-1,ch] f32, norm_w [dv] f32.
    Returns (out bf16 [B,T,Hv*dv], state_after, conv_state_after)."""
    if scale is None:
        scale = 1.0 / np.sqrt(dk)
    qkv, z, a, b, conv_w = (_c(x, U16) for x in (qkv, z, a, b, conv_w))
    dt_bias, A_log, norm_w = _c(dt_bias, U16), _c(A_log, F32), _c(norm_w, F32)
    st = np.array(state, dtype=F32, copy=True, order="C")
    cs = np.array(conv_state, dtype=F32, copy=True, order="C")
    ch = 2 * Hk * dk + Hv * dv
    out = np.zeros((B, T, Hv * dv), U16)
    lib(fast).orc_deltanet_layer(_p(qkv), ch, _p(z), Hv * dv, _p(a), _p(b), Hv, _p(conv_w), _p(cs),
                                 int(conv_head), _p(dt_bias), _p(A_log), _p(norm_w), _p(st), _p(out),
                                 B, T, Hk, Hv, dk, dv, K, eps, scale)
    return out, st, cs


def deltanet_recurrent_f64(q, k, v, a, b, state, B, T, Hk, Hv, dk, dv, eps=1e-6,
                           scale=None, l2norm=True, dt_bias=None, A_log=None):
    if scale is None:
        scale = 1.0 / np.sqrt(dk)
    q, k, v, a, b = (_c(x, U16) for x in (q, k, v, a, b))
    dt_bias, A_log = _c(dt_bias, U16), _c(A_log, F32)
    st = np.array(state, dtype=np.float64, copy=True, order="C")
    out = np.zeros((B, T, Hv, dv), np.float64)
    lib().orc_deltanet_recurrent_f64(_p(q), _p(k), _p(v), _p(a), _p(b), _p(dt_bias), _p(A_log),
                                     _p(st), _p(out), B, T, Hk, Hv, dk, dv, eps, scale, int(l2norm))
    return out, st


def num_threads(fast=False) -> int:
    return lib(fast).orc_num_threads()


def set_num_threads(n: int, fast=False) -> None:
    lib(fast).orc_set_num_threads(n)
