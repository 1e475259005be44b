"""Writes tests/golden/fixtures.npz: small input/output vectors of the path.

The reference holds no golden vectors for this path, so these are produced
by this repository's CPU oracle (``oracle/``, a scalar restatement of the
reference's functions) from the repository's seeded generator
(``aila_amd.datagen``: splitmix64 -> Box-Muller). Inputs are not stored:
each case names its seed, and the fixture records a checksum of the
generated inputs so that a change to the generator is caught as well.

Cases (reference functions they follow):
  decode128   attention_decode_baseline, AttentionOps.cpp:73-166
              B=2 Hq=8 Hkv=2 D=128 L=64
  decode256   the same at D=256 (the split-K path's head size), B=1
              Hq=16 Hkv=4 L=80
  prefill64   attention_prefill naive branch, AttentionOps.cpp:769-841,
              S=64 Hq=4 Hkv=2 D=64, causal
  cached128   attention_prefill_cached, AttentionOps.cpp:2308-2507,
              S=16 new rows after 48, Hq=4 Hkv=2 D=128
  deltanet    the gated delta recurrence, Qwen35HybridTextBackend.cpp:
              1729-1780 (q, k L2-normed, scale 1/sqrt(dk)), B=1 T=16 Hk=2
              Hv=4 dk=dv=128, state ~ N(0, 0.02^2); outputs of every step,
              the final state's sum and max |x| and every 97th value
  layer       the whole DeltaNet layer, Qwen35HybridTextBackend.cpp:
              1640-1798 (conv ring + SiLU, norms, recurrence, gated
              RMSNorm), B=1 T=8 Hk=2 Hv=4 d=128, ring head 1; outputs, the
              final state's summary as above and the final conv ring

Run from the repository root: ``python tests/golden/make_fixtures.py``.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from aila_amd import datagen as dg  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fixtures.npz")
SEED = 0xA11A + 100
STATE_STRIDE = 97


def checksum(*arrays) -> np.ndarray:
    """Order-dependent 64-bit checksum of raw array bytes."""
    h = np.uint64(1469598103934665603)
    for a in arrays:
        b = np.ascontiguousarray(a).reshape(-1).view(np.uint8).astype(np.uint64)
        w = np.arange(1, b.size + 1, dtype=np.uint64)
        h = np.uint64((int(h) * 1099511628211 + int(np.sum(b * w, dtype=np.uint64))) % (1 << 64))
    return np.array([h], dtype=np.uint64)


def state_summary(st: np.ndarray):
    flat = st.reshape(-1)
    return (np.array([np.sum(flat, dtype=np.float64), np.max(np.abs(flat))], dtype=np.float64),
            flat[::STATE_STRIDE].copy())


# ---- inputs (shared with the tests that read the fixture) -----------------
def decode_inputs(seed, B, Hq, Hkv, D, L):
    return (dg.normal_bf16(seed, 0, (B, Hq, D)), dg.normal_bf16(seed, 1, (B, Hkv, L, D)),
            dg.normal_bf16(seed, 2, (B, Hkv, L, D)))


def prefill_inputs(seed, S, Hq, Hkv, D):
    return (dg.normal_bf16(seed, 0, (S, Hq * D)), dg.normal_bf16(seed, 1, (S, Hkv * D)),
            dg.normal_bf16(seed, 2, (S, Hkv * D)))


def cached_inputs(seed, S, start, Hq, Hkv, D, max_seq):
    return (dg.normal_bf16(seed, 0, (S, Hq * D)), dg.normal_bf16(seed, 1, (Hkv, max_seq, D)),
            dg.normal_bf16(seed, 2, (Hkv, max_seq, D)))


def deltanet_inputs(seed, B, T, Hk, Hv, d):
    return dict(q=dg.normal_bf16(seed, 0, (B, T, Hk, d)), k=dg.normal_bf16(seed, 1, (B, T, Hk, d)),
                v=dg.normal_bf16(seed, 2, (B, T, Hv, d)), a=dg.normal_bf16(seed, 3, (B, T, Hv)),
                b=dg.normal_bf16(seed, 4, (B, T, Hv)),
                state=dg.normal(seed, 5, B * Hv * d * d, std=0.02).reshape(B, Hv, d, d).astype(np.float32))


def layer_inputs(seed, B, T, Hk, Hv, d):
    ch = 2 * Hk * d + Hv * d
    return dict(qkv=dg.normal_bf16(seed, 0, (B, T, ch)), z=dg.normal_bf16(seed, 1, (B, T, Hv * d)),
                a=dg.normal_bf16(seed, 2, (B, T, Hv)), b=dg.normal_bf16(seed, 3, (B, T, Hv)),
                conv_w=dg.normal_bf16(seed, 4, (ch, 4), std=0.5),
                conv_state=dg.normal(seed, 5, B * 3 * ch).reshape(B, 3, ch).astype(np.float32),
                norm_w=(1.0 + dg.normal(seed, 6, d, std=0.1)).astype(np.float32),
                state=dg.normal(seed, 7, B * Hv * d * d, std=0.02).reshape(B, Hv, d, d).astype(np.float32),
                dt_bias=dg.normal_bf16(seed, 8, (Hv,)),
                A_log=np.log(1.0 + np.abs(dg.normal(seed, 9, Hv, std=4.0))).astype(np.float32))


CASES = {
    "decode128": dict(seed=SEED + 1, B=2, Hq=8, Hkv=2, D=128, L=64),
    "decode256": dict(seed=SEED + 2, B=1, Hq=16, Hkv=4, D=256, L=80),
    "prefill64": dict(seed=SEED + 3, S=64, Hq=4, Hkv=2, D=64),
    "cached128": dict(seed=SEED + 4, S=16, start=48, Hq=4, Hkv=2, D=128, max_seq=64),
    "deltanet": dict(seed=SEED + 5, B=1, T=16, Hk=2, Hv=4, d=128),
    "layer": dict(seed=SEED + 6, B=1, T=8, Hk=2, Hv=4, d=128, head=1),
}


def compute() -> dict:
    f = {}
    for name in ("decode128", "decode256"):
        c = CASES[name]
        q, kc, vc = decode_inputs(c["seed"], c["B"], c["Hq"], c["Hkv"], c["D"], c["L"])
        f[f"{name}/inputs"] = checksum(q, kc, vc)
        f[f"{name}/out"] = oracle.attention_decode_baseline(q, kc, vc, c["B"], c["Hq"], c["Hkv"], c["D"],
                                                            c["L"], c["L"])
    c = CASES["prefill64"]
    q, k, v = prefill_inputs(c["seed"], c["S"], c["Hq"], c["Hkv"], c["D"])
    f["prefill64/inputs"] = checksum(q, k, v)
    f["prefill64/out"] = oracle.attention_prefill_naive(q, k, v, c["S"], c["Hq"], c["Hkv"], c["D"])
    c = CASES["cached128"]
    q, kc, vc = cached_inputs(c["seed"], c["S"], c["start"], c["Hq"], c["Hkv"], c["D"], c["max_seq"])
    f["cached128/inputs"] = checksum(q, kc, vc)
    f["cached128/out"] = oracle.attention_prefill_cached(q, kc, vc, c["S"], c["start"], c["Hq"], c["Hkv"],
                                                         c["D"], c["max_seq"])
    c = CASES["deltanet"]
    x = deltanet_inputs(c["seed"], c["B"], c["T"], c["Hk"], c["Hv"], c["d"])
    f["deltanet/inputs"] = checksum(*x.values())
    _, outb, st = oracle.deltanet_recurrent(x["q"], x["k"], x["v"], x["a"], x["b"], x["state"], c["B"], c["T"],
                                            c["Hk"], c["Hv"], c["d"], c["d"])
    f["deltanet/out"] = outb
    f["deltanet/state_stats"], f["deltanet/state_sample"] = state_summary(st)
    c = CASES["layer"]
    x = layer_inputs(c["seed"], c["B"], c["T"], c["Hk"], c["Hv"], c["d"])
    f["layer/inputs"] = checksum(*x.values())
    out, st, cs = oracle.deltanet_layer(x["qkv"], x["z"], x["a"], x["b"], x["conv_w"], x["conv_state"],
                                        c["head"], x["norm_w"], x["state"], c["B"], c["T"], c["Hk"], c["Hv"],
                                        c["d"], c["d"], dt_bias=x["dt_bias"], A_log=x["A_log"])
    f["layer/out"] = out
    f["layer/state_stats"], f["layer/state_sample"] = state_summary(st)
    f["layer/conv_state"] = cs
    return f


if __name__ == "__main__":
    fx = compute()
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT}: {len(fx)} arrays, {os.path.getsize(OUT)} bytes")
