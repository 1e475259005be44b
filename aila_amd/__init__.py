"""MI355X-native attention hot path for Aila (Qwen3 GQA + Gated DeltaNet).

The compute lives in ``aila_amd/libaila_hip.so`` (hand-written gfx950 HIP
kernels behind the C ABI declared in ``include/aila_hip.h``). This module
is a thin host-side binding over that C ABI for torch device tensors: it
checks shapes, dtypes and contiguity on the host, then passes raw device
pointers and the current HIP stream. There is no fallback: if the library
is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import math
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaila_hip.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGS = {
    "aila_hip_last_error": ([], ctypes.c_char_p),
    "aila_hip_version": ([], _I),
    "aila_hip_gqa_decode_workspace_size": ([_I, _I, _I], _SZ),
    "aila_hip_gqa_decode": ([_P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _I, _P, _P], _I),
    "aila_hip_gqa_decode_window": ([_P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _I, _P, _I, _I, _I, _P], _I),
    "aila_hip_gqa_decode_paged": ([_P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _P, _I, _I, _P, _P], _I),
    "aila_hip_kv_append_paged": ([_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P], _I),
    "aila_hip_gqa_decode_noalloc_max_bytes": ([], _SZ),
    "aila_hip_gqa_decode_noalloc": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P], _I),
    "aila_hip_gqa_decode_append": ([_P, _P, _P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _I, _P, _P], _I),
    "aila_hip_gqa_decode_prepare_append": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I,
                                            _I, _F, _F, _I, _P, _P, _P], _I),
    "aila_hip_kv_append": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P], _I),
    "aila_hip_gqa_prefill": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "aila_hip_gqa_prefill_cached": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "aila_hip_gqa_prefill_cached_workspace_size": ([_I, _I, _I, _I, _I], _SZ),
    "aila_hip_gqa_prefill_cached_ws": ([_P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _I, _P], _I),
    "aila_hip_copy_to_cache": ([_P, _P, _I, _I, _I, _I, _I, _P], _I),
    "aila_hip_deltanet_decode": ([_P, _P, _P, _P, _P, _P, _P, _P, _P,
                                  _I, _I, _I, _I, _I, _F, _F, _P], _I),
    "aila_hip_deltanet_prefill_workspace_size": ([_I, _I, _I, _I, _I], _SZ),
    "aila_hip_deltanet_layer_prefill_workspace_size": ([_I, _I, _I, _I, _I, _I], _SZ),
    "aila_hip_deltanet_layer_prefill": ([_P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P, _SZ,
                                         _I, _I, _I, _I, _I, _I, _I, _F, _F, _P], _I),
    "aila_hip_deltanet_layer_decode": ([_P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P,
                                        _I, _I, _I, _I, _I, _I, _F, _F, _P, _P], _I),
    "aila_hip_decode_prepare_qkv": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                     _I, _I, _I, _I, _I, _I, _F, _F, _I, _P, _P, _P], _I),
    "aila_hip_head_rms_norm": ([_P, _P, _I, _I, _I, _F, _P], _I),
    "aila_hip_apply_rope": ([_P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P], _I),
    "aila_hip_sigmoid_mul": ([_P, _P, _P, ctypes.c_long, _P], _I),
    "aila_hip_deltanet_prefill": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ,
                                   _I, _I, _I, _I, _I, _I, _F, _F, _P], _I),
}


class AilaHipError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AilaHipError(
                f"{LIB_PATH} not found: build it with `python -m aila_amd.build`")
        l = ctypes.CDLL(LIB_PATH)
        for name, (argt, rest) in _SIGS.items():
            f = getattr(l, name)
            f.argtypes = argt
            f.restype = rest
        _lib = l
    return _lib


def exported_symbols():
    return list(_SIGS)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().aila_hip_last_error().decode(errors="replace")
        raise AilaHipError(f"{what} failed ({rc}): {msg}")


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t, dtype, shape, name, align=16):
    import torch
    if t is None:
        raise ValueError(f"{name} is required")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")
    del torch


class RopePos(ctypes.Structure):
    """``aila_hip_rope_pos``: rotary positions that differ from the cache row
    (text shift past the prompt and interleaved mRoPE streams, the reference's
    apply_rope_partial arguments). Build it with :func:`rope_pos`."""
    _fields_ = [("interleaved", _I), ("pos_t", _P), ("pos_h", _P), ("pos_w", _P),
                ("pos_stride", _I), ("prompt_pos_len", _I), ("text_pos_delta", _I),
                ("prompt_pos_lens", _P), ("text_pos_deltas", _P),
                ("mrope_section_t", _I), ("mrope_section_h", _I), ("mrope_section_w", _I),
                ("inv_freq", _P)]


def rope_pos(prompt_pos_len: int = 0, text_pos_delta: int = 0, pos_t=None, pos_h=None, pos_w=None,
             interleaved: bool = True, sections=(0, 0, 0), prompt_pos_lens=None, text_pos_deltas=None,
             inv_freq=None):
    """Rotary position record. pos_t/pos_h/pos_w: device int32 [P] (one prompt,
    shared by every sequence) or [B, P] (per sequence); prompt_pos_lens /
    text_pos_deltas: optional device int32 [B] overriding the scalars;
    inv_freq: optional device float32 [rotary_dim/2] table (pair d rotates by
    position * inv_freq[d])."""
    import torch
    rp = RopePos()
    rp.interleaved = int(bool(interleaved))
    rp.prompt_pos_len = int(prompt_pos_len)
    rp.text_pos_delta = int(text_pos_delta)
    rp.mrope_section_t, rp.mrope_section_h, rp.mrope_section_w = (int(x) for x in sections)
    keep = []
    streams = (pos_t, pos_h, pos_w)
    if any(t is not None for t in streams):
        if any(t is None for t in streams):
            raise ValueError("pos_t, pos_h and pos_w go together")
        shape = tuple(pos_t.shape)
        if len(shape) not in (1, 2):
            raise ValueError("position streams must be [P] or [B, P]")
        for t, name in zip(streams, ("pos_t", "pos_h", "pos_w")):
            _need(t, torch.int32, shape, name, align=4)
            keep.append(t)
        rp.pos_t, rp.pos_h, rp.pos_w = (t.data_ptr() for t in streams)
        rp.pos_stride = shape[1] if len(shape) == 2 else 0
    for t, name in ((prompt_pos_lens, "prompt_pos_lens"), (text_pos_deltas, "text_pos_deltas")):
        if t is not None:
            _need(t, torch.int32, tuple(t.shape), name, align=4)
            keep.append(t)
    if prompt_pos_lens is not None:
        rp.prompt_pos_lens = prompt_pos_lens.data_ptr()
    if text_pos_deltas is not None:
        rp.text_pos_deltas = text_pos_deltas.data_ptr()
    if inv_freq is not None:
        _need(inv_freq, torch.float32, tuple(inv_freq.shape), "inv_freq", align=4)
        keep.append(inv_freq)
        rp.inv_freq = inv_freq.data_ptr()
    rp._keep = keep   # the device arrays must outlive the launches that read them
    return rp


def _rope_arg(rope):
    return None if rope is None else ctypes.byref(rope)


# ----------------------------------------------------------------- GQA ----
def gqa_decode_workspace_size(B: int, Hq: int, D: int) -> int:
    return int(lib().aila_hip_gqa_decode_workspace_size(B, Hq, D))


def gqa_decode(q, k_cache, v_cache, cached_len: int, out=None, workspace=None,
               seq_lens=None, window=None, stream=None):
    """q [B,Hq,D] bf16; k_cache/v_cache [B,Hkv,max_seq,D] bf16 -> out [B,Hq,D].

    ``workspace``: uint8 device tensor of >= gqa_decode_workspace_size bytes
    enables split-K; None runs the single-pass kernel. ``seq_lens``: optional
    int32 [B] device tensor of per-sequence lengths (<= cached_len).
    ``window``: optional (window, window_start, sink) — the reference's
    decode window with attention sinks (window_start -1: max(512, window))."""
    import torch
    B, Hq, D = q.shape
    Hkv, max_seq = k_cache.shape[1], k_cache.shape[2]
    _need(q, torch.bfloat16, (B, Hq, D), "q")
    _need(k_cache, torch.bfloat16, (B, Hkv, max_seq, D), "k_cache")
    _need(v_cache, torch.bfloat16, (B, Hkv, max_seq, D), "v_cache")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.bfloat16, (B, Hq, D), "out")
    ws_bytes = 0
    if workspace is not None:
        if not workspace.is_cuda or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous device tensor")
        ws_bytes = workspace.numel() * workspace.element_size()
    if seq_lens is not None:
        _need(seq_lens, torch.int32, (B,), "seq_lens", align=4)
    if window is not None:
        w, ws0, sink = (int(x) for x in window)
        rc = lib().aila_hip_gqa_decode_window(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                              _ptr(workspace), ws_bytes, B, Hq, Hkv, D, max_seq,
                                              int(cached_len), _ptr(seq_lens), w, ws0, sink, _stream(stream))
        _check(rc, "aila_hip_gqa_decode_window")
        return out
    rc = lib().aila_hip_gqa_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                   _ptr(workspace), ws_bytes, B, Hq, Hkv, D, max_seq,
                                   int(cached_len), _ptr(seq_lens), _stream(stream))
    _check(rc, "aila_hip_gqa_decode")
    return out


def gqa_decode_paged(q, k_pages, v_pages, block_table, seq_lens, max_len: int, out=None, workspace=None,
                     stream=None):
    """Decode over a paged cache. q [B,Hq,D]; k_pages/v_pages [num_pages,Hkv,
    page_size,D] bf16; block_table int32 [B, max_pages]; seq_lens int32 [B]
    (each <= max_len) -> out [B,Hq,D]."""
    import torch
    B, Hq, D = q.shape
    num_pages, Hkv, page_size = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
    max_pages = block_table.shape[1]
    _need(q, torch.bfloat16, (B, Hq, D), "q")
    _need(k_pages, torch.bfloat16, (num_pages, Hkv, page_size, D), "k_pages")
    _need(v_pages, torch.bfloat16, (num_pages, Hkv, page_size, D), "v_pages")
    _need(block_table, torch.int32, (B, max_pages), "block_table", align=4)
    _need(seq_lens, torch.int32, (B,), "seq_lens", align=4)
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.bfloat16, (B, Hq, D), "out")
    ws_bytes = 0
    if workspace is not None:
        if not workspace.is_cuda or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous device tensor")
        ws_bytes = workspace.numel() * workspace.element_size()
    rc = lib().aila_hip_gqa_decode_paged(_ptr(q), _ptr(k_pages), _ptr(v_pages), _ptr(out), _ptr(workspace),
                                         ws_bytes, B, Hq, Hkv, D, page_size, _ptr(block_table), max_pages,
                                         int(max_len), _ptr(seq_lens), _stream(stream))
    _check(rc, "aila_hip_gqa_decode_paged")
    return out


def kv_append_paged(k_new, v_new, k_pages, v_pages, block_table, positions, stream=None):
    """k_new/v_new [B,Hkv,D] -> row positions[b] of sequence b in the page pool."""
    import torch
    num_pages, Hkv, page_size, D = k_pages.shape
    B, max_pages = block_table.shape
    _need(k_new, torch.bfloat16, (B, Hkv, D), "k_new")
    _need(v_new, torch.bfloat16, (B, Hkv, D), "v_new")
    _need(k_pages, torch.bfloat16, (num_pages, Hkv, page_size, D), "k_pages")
    _need(v_pages, torch.bfloat16, (num_pages, Hkv, page_size, D), "v_pages")
    _need(block_table, torch.int32, (B, max_pages), "block_table", align=4)
    _need(positions, torch.int32, (B,), "positions", align=4)
    rc = lib().aila_hip_kv_append_paged(_ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages), B, Hkv, D,
                                        page_size, _ptr(block_table), max_pages, _ptr(positions), _stream(stream))
    _check(rc, "aila_hip_kv_append_paged")


def gqa_decode_noalloc(q, k_cache, v_cache, cached_len: int, out=None, seq_lens=None, stream=None):
    """gqa_decode with the split records in the library's static device
    scratch (no workspace argument, no allocation in the library). Calls
    that overlap on one GPU share that scratch and race."""
    import torch
    B, Hq, D = q.shape
    Hkv, max_seq = k_cache.shape[1], k_cache.shape[2]
    _need(q, torch.bfloat16, (B, Hq, D), "q")
    _need(k_cache, torch.bfloat16, (B, Hkv, max_seq, D), "k_cache")
    _need(v_cache, torch.bfloat16, (B, Hkv, max_seq, D), "v_cache")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.bfloat16, (B, Hq, D), "out")
    if seq_lens is not None:
        _need(seq_lens, torch.int32, (B,), "seq_lens", align=4)
    rc = lib().aila_hip_gqa_decode_noalloc(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), B, Hq, Hkv, D,
                                           max_seq, int(cached_len), _ptr(seq_lens), _stream(stream))
    _check(rc, "aila_hip_gqa_decode_noalloc")
    return out


def gqa_decode_append(q, k_new, v_new, k_cache, v_cache, pos: int, out=None, workspace=None,
                      positions=None, stream=None):
    """Write k_new/v_new [B,Hkv,D] to cache row pos (or positions[b] <= pos)
    and attend rows [0, row] -> out [B,Hq,D]."""
    import torch
    B, Hq, D = q.shape
    Hkv, max_seq = k_cache.shape[1], k_cache.shape[2]
    _need(q, torch.bfloat16, (B, Hq, D), "q")
    _need(k_new, torch.bfloat16, (B, Hkv, D), "k_new")
    _need(v_new, torch.bfloat16, (B, Hkv, D), "v_new")
    _need(k_cache, torch.bfloat16, (B, Hkv, max_seq, D), "k_cache")
    _need(v_cache, torch.bfloat16, (B, Hkv, max_seq, D), "v_cache")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.bfloat16, (B, Hq, D), "out")
    ws_bytes = 0
    if workspace is not None:
        if not workspace.is_cuda or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous device tensor")
        ws_bytes = workspace.numel() * workspace.element_size()
    if positions is not None:
        _need(positions, torch.int32, (B,), "positions", align=4)
    rc = lib().aila_hip_gqa_decode_append(_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache),
                                          _ptr(out), _ptr(workspace), ws_bytes, B, Hq, Hkv, D, max_seq,
                                          int(pos), _ptr(positions), _stream(stream))
    _check(rc, "aila_hip_gqa_decode_append")
    return out


def kv_append(k_new, v_new, k_cache, v_cache, pos: int = 0, positions=None, stream=None):
    """k_new/v_new [B,Hkv,D] -> cache [B,Hkv,max_seq,D] row pos (or positions[b])."""
    import torch
    B, Hkv, max_seq, D = k_cache.shape
    _need(k_new, torch.bfloat16, (B, Hkv, D), "k_new")
    _need(v_new, torch.bfloat16, (B, Hkv, D), "v_new")
    _need(k_cache, torch.bfloat16, (B, Hkv, max_seq, D), "k_cache")
    _need(v_cache, torch.bfloat16, (B, Hkv, max_seq, D), "v_cache")
    if positions is not None:
        _need(positions, torch.int32, (B,), "positions", align=4)
    rc = lib().aila_hip_kv_append(_ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), B, Hkv, D,
                                  max_seq, int(pos), _ptr(positions), _stream(stream))
    _check(rc, "aila_hip_kv_append")


def gqa_prefill(q, k, v, Hq: int, Hkv: int, out=None, k_cache=None, v_cache=None,
                cache_pos: int = 0, stream=None):
    """Causal prefill. q [S, Hq*D], k/v [S, Hkv*D] bf16 -> out [S, Hq*D].
    With k_cache/v_cache [Hkv, max_seq, D], k/v are also written to cache
    rows [cache_pos, cache_pos + S)."""
    import torch
    S = q.shape[0]
    D = q.shape[1] // Hq
    _need(q, torch.bfloat16, (S, Hq * D), "q")
    _need(k, torch.bfloat16, (S, Hkv * D), "k")
    _need(v, torch.bfloat16, (S, Hkv * D), "v")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.bfloat16, (S, Hq * D), "out")
    max_seq = 0
    if k_cache is not None or v_cache is not None:
        max_seq = k_cache.shape[1]
        _need(k_cache, torch.bfloat16, (Hkv, max_seq, D), "k_cache")
        _need(v_cache, torch.bfloat16, (Hkv, max_seq, D), "v_cache")
    rc = lib().aila_hip_gqa_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(k_cache),
                                    _ptr(v_cache), int(cache_pos), max_seq, S, Hq, Hkv, D,
                                    _stream(stream))
    _check(rc, "aila_hip_gqa_prefill")
    return out


def gqa_prefill_cached_workspace_size(S: int, start_pos: int, Hq: int, Hkv: int, D: int) -> int:
    """Bytes of the key-split workspace gqa_prefill_cached would use (0: none)."""
    return int(lib().aila_hip_gqa_prefill_cached_workspace_size(S, start_pos, Hq, Hkv, D))


def gqa_prefill_cached(q, k_cache, v_cache, start_pos: int, Hq: int, out=None, workspace=None, stream=None):
    """q [S, Hq*D] at positions start_pos.. attends cache [Hkv, max_seq, D].
    workspace: a uint8 device tensor for the key split (see
    gqa_prefill_cached_workspace_size), or None for no split."""
    import torch
    S = q.shape[0]
    Hkv, max_seq, D = k_cache.shape
    _need(q, torch.bfloat16, (S, Hq * D), "q")
    _need(k_cache, torch.bfloat16, (Hkv, max_seq, D), "k_cache")
    _need(v_cache, torch.bfloat16, (Hkv, max_seq, D), "v_cache")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.bfloat16, (S, Hq * D), "out")
    if workspace is None:
        rc = lib().aila_hip_gqa_prefill_cached(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), S,
                                               int(start_pos), Hq, Hkv, D, max_seq, _stream(stream))
    else:
        if not workspace.is_cuda or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous device tensor")
        rc = lib().aila_hip_gqa_prefill_cached_ws(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                                  _ptr(workspace), workspace.numel() * workspace.element_size(),
                                                  S, int(start_pos), Hq, Hkv, D, max_seq, _stream(stream))
    _check(rc, "aila_hip_gqa_prefill_cached")
    return out


def copy_to_cache(new_kv, cache, start_pos: int, stream=None):
    """new_kv [S, H*D] bf16 -> cache [H, max_seq, D] rows [start_pos, start_pos+S)."""
    import torch
    H, max_seq, D = cache.shape
    S = new_kv.shape[0]
    _need(new_kv, torch.bfloat16, (S, H * D), "new_kv")
    _need(cache, torch.bfloat16, (H, max_seq, D), "cache")
    rc = lib().aila_hip_copy_to_cache(_ptr(new_kv), _ptr(cache), S, int(start_pos), H, D, max_seq,
                                      _stream(stream))
    _check(rc, "aila_hip_copy_to_cache")
    return cache


# ------------------------------------------------------------ DeltaNet ----
def deltanet_decode(q, k, v, a, b, state, out=None, dt_bias=None, A_log=None,
                    eps: float = 1e-6, scale: float | None = None, stream=None):
    """One Gated DeltaNet step. q,k [B,Hk,dk] bf16; v [B,Hv,dv] bf16;
    a,b [B,Hv] bf16; state [B,Hv,dk,dv] fp32 (updated in place) -> out
    [B,Hv,dv] bf16."""
    import torch
    B, Hk, dk = q.shape
    Hv, dv = v.shape[1], v.shape[2]
    _need(q, torch.bfloat16, (B, Hk, dk), "q")
    _need(k, torch.bfloat16, (B, Hk, dk), "k")
    _need(v, torch.bfloat16, (B, Hv, dv), "v")
    _need(a, torch.bfloat16, (B, Hv), "a", align=2)
    _need(b, torch.bfloat16, (B, Hv), "b", align=2)
    _need(state, torch.float32, (B, Hv, dk, dv), "state")
    if dt_bias is not None:
        _need(dt_bias, torch.bfloat16, (Hv,), "dt_bias", align=2)
    if A_log is not None:
        _need(A_log, torch.float32, (Hv,), "A_log", align=4)
    if out is None:
        out = torch.empty((B, Hv, dv), dtype=torch.bfloat16, device=q.device)
    _need(out, torch.bfloat16, (B, Hv, dv), "out")
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    rc = lib().aila_hip_deltanet_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
                                        _ptr(dt_bias), _ptr(A_log), _ptr(state), _ptr(out),
                                        B, Hk, Hv, dk, dv, float(eps), float(scale),
                                        _stream(stream))
    _check(rc, "aila_hip_deltanet_decode")
    return out


def _rows(t, dtype, B, width, name, align=2):
    """A [B, width] view whose rows may be strided (e.g. column slices of the
    backend's fused [qkv | z | a | b] rows); returns the row stride."""
    if t is None or not t.is_cuda or t.dtype != dtype:
        raise ValueError(f"{name}: expected a {dtype} device tensor")
    if t.dim() != 2 or tuple(t.shape) != (B, width) or (width > 1 and t.stride(1) != 1):
        raise ValueError(f"{name}: shape {tuple(t.shape)} / strides {t.stride()}, expected [{B}, {width}] "
                         "with unit column stride")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")
    return t.stride(0) if B > 1 else width


def deltanet_layer_decode(qkv, z, a, b, conv_w, conv_state, conv_head, norm_w, state, num_k_heads,
                          out=None, conv_heads=None, dt_bias=None, A_log=None, eps: float = 1e-6,
                          scale: float | None = None, arrivals=None, stream=None):
    """Full Gated DeltaNet layer step for B sequences: conv1d ring (+SiLU),
    L2 norm, gated delta recurrence, RMSNorm(o) * norm_w * SiLU(z).

    qkv [B, 2*Hk*dk + Hv*dv], z [B, Hv*dv], a/b [B, Hv] bf16 (rows may be
    strided views); conv_w [ch, 4] bf16; conv_state [B, 3, ch] fp32 and
    state [B, Hv, dk, dv] fp32 are updated in place; conv_head (int) or
    conv_heads (int32 [B], device) gives the ring row of the oldest input.
    ``arrivals``: optional int32 [B*Hk] device tensor, zero before the first
    call (every call leaves it zero): one workgroup per value head instead
    of one per key head. Returns out [B, Hv*dv] bf16."""
    import torch
    B, Hv, dk, dv = state.shape
    Hk = int(num_k_heads)
    ch = 2 * Hk * dk + Hv * dv
    qs = _rows(qkv, torch.bfloat16, B, ch, "qkv")
    zs = _rows(z, torch.bfloat16, B, Hv * dv, "z", align=8)
    ast = _rows(a, torch.bfloat16, B, Hv, "a")
    bst = _rows(b, torch.bfloat16, B, Hv, "b")
    if ast != bst:
        raise ValueError("a and b must share one row stride")
    K = conv_w.shape[1]
    _need(conv_w, torch.bfloat16, (ch, K), "conv_w", align=8)
    _need(conv_state, torch.float32, (B, K - 1, ch), "conv_state", align=4)
    _need(norm_w, torch.float32, (dv,), "norm_w")
    _need(state, torch.float32, (B, Hv, dk, dv), "state")
    if conv_heads is not None:
        _need(conv_heads, torch.int32, (B,), "conv_heads", align=4)
    if dt_bias is not None:
        _need(dt_bias, torch.bfloat16, (Hv,), "dt_bias", align=2)
    if A_log is not None:
        _need(A_log, torch.float32, (Hv,), "A_log", align=4)
    if out is None:
        out = torch.empty((B, Hv * dv), dtype=torch.bfloat16, device=state.device)
    _need(out, torch.bfloat16, (B, Hv * dv), "out", align=8)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    if arrivals is not None:
        _need(arrivals, torch.int32, (B * Hk,), "arrivals", align=4)
    rc = lib().aila_hip_deltanet_layer_decode(
        _ptr(qkv), qs, _ptr(z), zs, _ptr(a), _ptr(b), ast, _ptr(conv_w), _ptr(conv_state), int(conv_head),
        _ptr(conv_heads), _ptr(dt_bias), _ptr(A_log), _ptr(norm_w), _ptr(state), _ptr(out), B, Hk, Hv, dk, dv,
        K, float(eps), float(scale), _ptr(arrivals), _stream(stream))
    _check(rc, "aila_hip_deltanet_layer_decode")
    return out


def _tok_rows(t, dtype, B, T, width, name, align=2):
    """A [B, T, width] view whose token rows may be strided (column slices of
    fused rows); the rows of all sequences must be equally spaced."""
    if t is None or not t.is_cuda or t.dtype != dtype:
        raise ValueError(f"{name}: expected a {dtype} device tensor")
    if t.dim() != 3 or tuple(t.shape) != (B, T, width) or (width > 1 and t.stride(2) != 1):
        raise ValueError(f"{name}: shape {tuple(t.shape)} / strides {t.stride()}, expected [{B}, {T}, {width}]")
    rs = t.stride(1) if T > 1 else (t.stride(0) if B > 1 else width)
    if B > 1 and t.stride(0) != T * rs:
        raise ValueError(f"{name}: sequences must follow each other (stride(0) = T * stride(1))")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")
    return rs


def deltanet_layer_prefill_workspace_size(B: int, T: int, Hk: int, Hv: int, dk: int = 128, dv: int = 128) -> int:
    return int(lib().aila_hip_deltanet_layer_prefill_workspace_size(B, T, Hk, Hv, dk, dv))


def deltanet_layer_prefill(qkv, z, a, b, conv_w, conv_state, conv_head, norm_w, state, num_k_heads,
                           out=None, workspace=None, dt_bias=None, A_log=None, eps: float = 1e-6,
                           scale: float | None = None, stream=None):
    """Full Gated DeltaNet layer over T tokens: qkv [B,T,ch], z [B,T,Hv*dv],
    a/b [B,T,Hv] bf16 (token rows may be strided views of fused rows);
    conv_state [B,3,ch] and state [B,Hv,dk,dv] fp32 updated in place.
    Returns out [B,T,Hv*dv] bf16; the caller advances conv_head by T."""
    import torch
    B, Hv, dk, dv = state.shape
    T = qkv.shape[1]
    Hk = int(num_k_heads)
    ch = 2 * Hk * dk + Hv * dv
    qs = _tok_rows(qkv, torch.bfloat16, B, T, ch, "qkv", align=8)
    zs = _tok_rows(z, torch.bfloat16, B, T, Hv * dv, "z", align=16)
    ast = _tok_rows(a, torch.bfloat16, B, T, Hv, "a")
    bst = _tok_rows(b, torch.bfloat16, B, T, Hv, "b")
    if ast != bst:
        raise ValueError("a and b must share one row stride")
    K = conv_w.shape[1]
    _need(conv_w, torch.bfloat16, (ch, K), "conv_w")
    _need(conv_state, torch.float32, (B, K - 1, ch), "conv_state")
    _need(norm_w, torch.float32, (dv,), "norm_w", align=16)
    _need(state, torch.float32, (B, Hv, dk, dv), "state")
    if dt_bias is not None:
        _need(dt_bias, torch.bfloat16, (Hv,), "dt_bias", align=2)
    if A_log is not None:
        _need(A_log, torch.float32, (Hv,), "A_log", align=4)
    if out is None:
        out = torch.empty((B, T, Hv * dv), dtype=torch.bfloat16, device=state.device)
    _need(out, torch.bfloat16, (B, T, Hv * dv), "out")
    need = deltanet_layer_prefill_workspace_size(B, T, Hk, Hv, dk, dv)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=state.device)
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    rc = lib().aila_hip_deltanet_layer_prefill(
        _ptr(qkv), qs, _ptr(z), zs, _ptr(a), _ptr(b), ast, _ptr(conv_w), _ptr(conv_state), int(conv_head),
        _ptr(dt_bias), _ptr(A_log), _ptr(norm_w), _ptr(state), _ptr(out), _ptr(workspace),
        workspace.numel() * workspace.element_size(), B, T, Hk, Hv, dk, dv, K, float(eps), float(scale),
        _stream(stream))
    _check(rc, "aila_hip_deltanet_layer_prefill")
    return out


def deltanet_prefill_workspace_size(B: int, T: int, Hv: int, dk: int, dv: int) -> int:
    return int(lib().aila_hip_deltanet_prefill_workspace_size(B, T, Hv, dk, dv))


def deltanet_prefill(q, k, v, a, b, state, out=None, workspace=None, dt_bias=None,
                     A_log=None, eps: float = 1e-6, scale: float | None = None, stream=None):
    """Chunked prefill over T tokens. q,k [B,T,Hk,dk]; v [B,T,Hv,dv]; a,b
    [B,T,Hv] bf16; state [B,Hv,dk,dv] fp32 (in/out) -> out [B,T,Hv,dv] bf16.
    ``workspace``: uint8 device tensor (allocated here when None)."""
    import torch
    B, T, Hk, dk = q.shape
    Hv, dv = v.shape[2], v.shape[3]
    _need(q, torch.bfloat16, (B, T, Hk, dk), "q")
    _need(k, torch.bfloat16, (B, T, Hk, dk), "k")
    _need(v, torch.bfloat16, (B, T, Hv, dv), "v")
    _need(a, torch.bfloat16, (B, T, Hv), "a", align=2)
    _need(b, torch.bfloat16, (B, T, Hv), "b", align=2)
    _need(state, torch.float32, (B, Hv, dk, dv), "state")
    if dt_bias is not None:
        _need(dt_bias, torch.bfloat16, (Hv,), "dt_bias", align=2)
    if A_log is not None:
        _need(A_log, torch.float32, (Hv,), "A_log", align=4)
    if out is None:
        out = torch.empty((B, T, Hv, dv), dtype=torch.bfloat16, device=q.device)
    _need(out, torch.bfloat16, (B, T, Hv, dv), "out")
    need = deltanet_prefill_workspace_size(B, T, Hv, dk, dv)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size()
    if scale is None:
        scale = 1.0 / math.sqrt(dk)
    rc = lib().aila_hip_deltanet_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
                                         _ptr(dt_bias), _ptr(A_log), _ptr(state), _ptr(out),
                                         _ptr(workspace), ws_bytes, B, T, Hk, Hv, dk, dv,
                                         float(eps), float(scale), _stream(stream))
    _check(rc, "aila_hip_deltanet_prefill")
    return out


# ------------------------------------------ QK-norm, RoPE, output gate ----
def decode_prepare_qkv(q_in, k, v, q_norm_w=None, k_norm_w=None, k_cache=None, v_cache=None,
                       pos: int = 0, positions=None, rotary_dim=None, theta: float = 1e6,
                       eps: float = 1e-6, packed_gate: bool = False, q_out=None, gate_out=None,
                       rope=None, stream=None):
    """Per-head RMSNorm + RoPE of one token per sequence, and the K/V append.

    q_in [B,Hq,D] (or [B,Hq,2D] q|gate when ``packed_gate``); k [B,Hkv,D] is
    updated in place; v [B,Hkv,D]; caches [B,Hkv,max_seq,D] or None. Returns
    q_out (and gate_out when packed). rope: a :func:`rope_pos` record (text
    shift / mRoPE positions); None rotates at the cache row."""
    import torch
    B, Hkv, D = k.shape
    Hq = q_in.shape[1]
    _need(q_in, torch.bfloat16, (B, Hq, 2 * D if packed_gate else D), "q_in")
    _need(k, torch.bfloat16, (B, Hkv, D), "k")
    _need(v, torch.bfloat16, (B, Hkv, D), "v")
    if q_out is None:
        q_out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=k.device) if packed_gate else q_in
    _need(q_out, torch.bfloat16, (B, Hq, D), "q_out")
    if packed_gate:
        if gate_out is None:
            gate_out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=k.device)
        _need(gate_out, torch.bfloat16, (B, Hq, D), "gate_out")
    for w, name in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
        if w is not None:
            _need(w, torch.bfloat16, (D,), name, align=2)
    max_seq = 0
    if k_cache is not None or v_cache is not None:
        max_seq = k_cache.shape[2]
        _need(k_cache, torch.bfloat16, (B, Hkv, max_seq, D), "k_cache")
        _need(v_cache, torch.bfloat16, (B, Hkv, max_seq, D), "v_cache")
    if positions is not None:
        _need(positions, torch.int32, (B,), "positions", align=4)
    rc = lib().aila_hip_decode_prepare_qkv(
        _ptr(q_in), int(bool(packed_gate)), _ptr(q_out), _ptr(gate_out) if packed_gate else None,
        _ptr(k), _ptr(v), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(k_cache), _ptr(v_cache), B, Hq, Hkv, D,
        max_seq, D if rotary_dim is None else int(rotary_dim), float(theta), float(eps), int(pos),
        _ptr(positions), _rope_arg(rope), _stream(stream))
    _check(rc, "decode_prepare_qkv")
    return (q_out, gate_out) if packed_gate else q_out


def gqa_decode_prepare_append(q_in, k_new, v_new, k_cache, v_cache, pos: int, q_norm_w=None, k_norm_w=None,
                              rotary_dim=None, theta: float = 1e6, eps: float = 1e-6, packed_gate: bool = False,
                              out=None, gate_out=None, workspace=None, positions=None, apply_gate: bool = False,
                              rope=None, stream=None):
    """QK-norm + RoPE + K/V append + split-K decode in one launch.
    q_in [B,Hq,D] (or [B,Hq,2D] q|gate when packed_gate); k_new/v_new [B,Hkv,D];
    caches [B,Hkv,max_seq,D]. Returns out (and gate_out when packed).
    apply_gate (packed only): out = attention * sigmoid(gate), the gated
    attention epilogue, instead of returning the gate.
    Without a workspace the decode runs single-pass (one workgroup per KV
    head), as gqa_decode_append."""
    import torch
    if apply_gate and not packed_gate:
        raise ValueError("apply_gate needs packed_gate")
    B, Hkv, max_seq, D = k_cache.shape
    Hq = q_in.shape[1]
    _need(q_in, torch.bfloat16, (B, Hq, 2 * D if packed_gate else D), "q_in")
    _need(k_new, torch.bfloat16, (B, Hkv, D), "k_new")
    _need(v_new, torch.bfloat16, (B, Hkv, D), "v_new")
    _need(k_cache, torch.bfloat16, (B, Hkv, max_seq, D), "k_cache")
    _need(v_cache, torch.bfloat16, (B, Hkv, max_seq, D), "v_cache")
    for w, name in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
        if w is not None:
            _need(w, torch.bfloat16, (D,), name, align=2)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=k_cache.device)
    _need(out, torch.bfloat16, (B, Hq, D), "out")
    if packed_gate and not apply_gate:
        if gate_out is None:
            gate_out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=k_cache.device)
        _need(gate_out, torch.bfloat16, (B, Hq, D), "gate_out")
    ws_bytes = 0
    if workspace is not None:
        if not workspace.is_cuda or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous device tensor")
        ws_bytes = workspace.numel() * workspace.element_size()
    if positions is not None:
        _need(positions, torch.int32, (B,), "positions", align=4)
    rc = lib().aila_hip_gqa_decode_prepare_append(
        _ptr(q_in), 2 if apply_gate else int(bool(packed_gate)), _ptr(gate_out) if packed_gate and not apply_gate else None,
        _ptr(k_new), _ptr(v_new),
        _ptr(q_norm_w), _ptr(k_norm_w), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(workspace),
        ws_bytes, B, Hq, Hkv, D, max_seq,
        D if rotary_dim is None else int(rotary_dim), float(theta), float(eps), int(pos), _ptr(positions),
        _rope_arg(rope), _stream(stream))
    _check(rc, "gqa_decode_prepare_append")
    return (out, gate_out) if packed_gate and not apply_gate else out


def head_rms_norm(x, weight=None, eps: float = 1e-6, stream=None):
    """In-place per-head RMSNorm of x [S, H, D] bf16 (weight [D] bf16 or None)."""
    import torch
    S, H, D = x.shape
    _need(x, torch.bfloat16, (S, H, D), "x")
    if weight is not None:
        _need(weight, torch.bfloat16, (D,), "weight", align=2)
    _check(lib().aila_hip_head_rms_norm(_ptr(x), _ptr(weight), S, H, D, float(eps), _stream(stream)),
           "head_rms_norm")
    return x


def apply_rope(q, k, start_pos: int = 0, rotary_dim=None, theta: float = 1e6, rope=None, stream=None):
    """In-place RoPE of q [S,Hq,D] and k [S,Hkv,D] bf16 for the tokens of cache
    rows start_pos + s (at those rows, or at the positions of ``rope``)."""
    import torch
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    _need(q, torch.bfloat16, (S, Hq, D), "q")
    _need(k, torch.bfloat16, (S, Hkv, D), "k")
    _check(lib().aila_hip_apply_rope(_ptr(q), _ptr(k), S, int(start_pos), Hq, Hkv, D,
                                     D if rotary_dim is None else int(rotary_dim), float(theta),
                                     _rope_arg(rope), _stream(stream)), "apply_rope")
    return q, k


def sigmoid_mul(inp, gate, out=None, stream=None):
    """out = inp * sigmoid(gate), bf16 tensors of equal shape (out may be inp)."""
    import torch
    if out is None:
        out = torch.empty_like(inp)
    for t, name in ((inp, "input"), (gate, "gate"), (out, "output")):
        _need(t, torch.bfloat16, tuple(inp.shape), name)
    _check(lib().aila_hip_sigmoid_mul(_ptr(inp), _ptr(gate), _ptr(out), inp.numel(), _stream(stream)),
           "sigmoid_mul")
    return out
