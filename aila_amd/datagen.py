"""Deterministic synthetic inputs and bf16 helpers (host side, numpy).

The generator is counter based so any host (and the GPU fill kernel in
``aila_amd/csrc/fill.hip``) can reproduce a tensor from ``(seed, stream)``:

  * ``mix(x)`` is the splitmix64 finaliser; element pair ``p`` of stream ``s``
    uses words ``mix(key + (2p+1)*G)`` and ``mix(key + (2p+2)*G)`` with
    ``key = mix(seed ^ (s * 0xD1B54A32D192ED03))`` and ``G = 0x9E3779B97F4A7C15``.
  * Uniforms: ``u1 = ((x1 >> 11) + 0.5) * 2^-53`` (never 0), ``u2 = (x2 >> 11) * 2^-53``.
  * Box-Muller in fp64: ``r = sqrt(-2 ln u1)``, ``z0 = r cos(2 pi u2)``,
    ``z1 = r sin(2 pi u2)``; values are rounded to fp32.

Seeds are ``0xA11A + config_index`` for the benchmark configs; each tensor of
a config draws its own stream index in a fixed order.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
STREAM_MUL = np.uint64(0xD1B54A32D192ED03)
SEED_BASE = 0xA11A


def _mix(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    return x


def stream_key(seed: int, stream: int) -> np.uint64:
    with np.errstate(over="ignore"):
        v = np.uint64(seed) ^ (np.uint64(stream) * STREAM_MUL)
    return _mix(np.array([v], dtype=np.uint64))[0]


def normal(seed: int, stream: int, n: int, std: float = 1.0) -> np.ndarray:
    """n fp32 samples of N(0, std^2) from (seed, stream)."""
    npairs = (n + 1) // 2
    key = stream_key(seed, stream)
    p = np.arange(npairs, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x1 = _mix(key + (np.uint64(2) * p + np.uint64(1)) * GOLDEN)
        x2 = _mix(key + (np.uint64(2) * p + np.uint64(2)) * GOLDEN)
    u1 = ((x1 >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)
    u2 = (x2 >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    r = np.sqrt(-2.0 * np.log(u1))
    th = 2.0 * np.pi * u2
    out = np.empty(2 * npairs, dtype=np.float64)
    out[0::2] = r * np.cos(th)
    out[1::2] = r * np.sin(th)
    out = out[:n]
    if std != 1.0:
        out = out * std
    return out.astype(np.float32)


# ----------------------------------------------------------------- bf16 ----
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (uint16); NaN stays quiet NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    lsb = (u >> 16) & 1
    r = ((u + np.uint32(0x7FFF) + lsb) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded through bf16 (returned as fp32)."""
    return bf16_to_f32(f32_to_bf16(x))


def normal_bf16(seed: int, stream: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return f32_to_bf16(normal(seed, stream, n, std)).reshape(shape)


# ------------------------------------------------------ input builders ----
def rms_norm_rows_bf16(x_bf16: np.ndarray, D: int, eps: float = 1e-6) -> np.ndarray:
    """Per-head RMSNorm with unit weight and bf16 rounding (head_rms_norm,
    NormOps.cpp:277-321): rows of length D, sum of squares in fp32."""
    x = bf16_to_f32(x_bf16).reshape(-1, D)
    ss = np.zeros(x.shape[0], dtype=np.float32)
    for d in range(D):  # sequential fp32 sum, the reference's per-lane order
        ss += x[:, d] * x[:, d]
    rms = np.sqrt(ss / np.float32(D) + np.float32(eps)).astype(np.float32)
    return f32_to_bf16(x / rms[:, None]).reshape(x_bf16.shape)
