#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline workload (benchmark config 5): decode of a Qwen3.5-4B-shaped hybrid
attention stack, 32 layers in a 3:1 pattern (24 Gated DeltaNet layers with
16 qk / 32 v heads, dk = dv = 128, fp32 state; 8 GQA layers with 16 q / 4 kv
heads, head_dim 256, bf16 KV cache), batch 8, context 32768, one new token
per step. A step is one token through all 32 layers: for each GQA layer the
new K/V row is appended and split-K decode runs over the cache (one fused
launch); for each
DeltaNet layer the state is updated once. value = algorithmic HBM bytes per
step / step time (GB/s). Steps are replayed from HIP graphs (device-side
lengths advance inside the graph), so host launch overhead is not timed.

Also reported (sub-metrics, same run): GQA prefill TFLOP/s (config 2),
DeltaNet decode us/step (config 3), DeltaNet chunked prefill tok/s
(config 4), GQA decode latency at config 1, the roofline of the dominant
kernel (GQA split-K decode, HIP events around each launch) and a CPU
baseline (the scalar oracle on the host cores, bounded sample).

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 8]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "GQA decode HBM GB/s @32k ctx; prefill MFMA TFLOP/s; DeltaNet tok/s (1 GPU)"

# config 5 shape
B5, L5 = 8, 32768
GQA_HQ, GQA_HKV, GQA_D = 16, 4, 256
DN_HK, DN_HV, DN_D = 16, 32, 128
N_LAYERS, N_GQA = 32, 8
NPOOL = 4   # distinct activation sets (one captured graph each)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gqa_bytes(B, Hq, Hkv, D, L):
    """Algorithmic bytes of one GQA decode launch: K and V rows read once,
    q read and out written once."""
    return 2 * B * Hkv * L * D * 2 + 2 * B * Hq * D * 2


def deltanet_bytes(B, Hk, Hv, dk, dv):
    """State read + write once, q,k,v,a,b read, out written."""
    return (2 * B * Hv * dk * dv * 4 + 2 * B * Hk * dk * 2 + B * Hv * dv * 2
            + 2 * B * Hv * 2 + B * Hv * dv * 2)


def deltanet_layer_bytes(B, Hk, Hv, d):
    """Full layer step: state read + write, conv ring 3 rows read + 1 written
    (fp32), the qkv row, z, a, b read, out written, conv_w read."""
    ch = 2 * Hk * d + Hv * d
    return (2 * B * Hv * d * d * 4 + 4 * B * ch * 4 + B * ch * 2 + B * Hv * d * 2 + 2 * B * Hv * 2
            + B * Hv * d * 2 + ch * 4 * 2)


def _drm_device_dir(torch):
    """sysfs directory of the DRM card that is torch device 0 (matched by
    PCI address), or None."""
    import glob
    try:
        pr = torch.cuda.get_device_properties(0)
        want = f"{pr.pci_domain_id:04x}:{pr.pci_bus_id:02x}:{pr.pci_device_id:02x}"
    except Exception:
        want = None
    cards = sorted(glob.glob("/sys/class/drm/card[0-9]*/device/pp_dpm_sclk"))
    for c in cards:
        d = os.path.dirname(c)
        if want and os.path.basename(os.path.realpath(d)).startswith(want):
            return d
    return os.path.dirname(cards[0]) if len(cards) == 1 else None


def _dpm_levels(path):
    """(MHz of the table's fixed levels, MHz of the current '*' line) of a
    pp_dpm file. The current line reads the actual clock: between levels
    the driver shows it as an extra starred entry, so starred entries are
    left out of the levels (a table with only a starred entry keeps it)."""
    levels, cur = [], None
    for line in open(path).read().splitlines():
        f = line.split()
        if len(f) < 2 or not f[1].lower().endswith("mhz"):
            continue
        mhz = int(float(f[1][:-3]))
        if line.rstrip().endswith("*"):
            cur = mhz
        elif not f[0].startswith("S"):
            levels.append(mhz)
    if not levels and cur is not None:
        levels = [cur]
    return sorted(levels), cur


class ClockSampler:
    """Samples the shader clock (the current pp_dpm_sclk level, which reads
    the actual frequency under load) and board power (hwmon power1_input)
    every ~5 ms from a host thread while active; sysfs reads only, so the
    GPU work is untouched."""

    def __init__(self, torch):
        import threading
        self.dev = _drm_device_dir(torch)
        self.sclk, self.power = [], []
        self._stop = threading.Event()
        self._t = None

    def _run(self):
        import glob
        pw = sorted(glob.glob(os.path.join(self.dev, "hwmon", "hwmon*", "power1_input")))
        while not self._stop.is_set():
            try:
                _, cur = _dpm_levels(os.path.join(self.dev, "pp_dpm_sclk"))
                if cur is not None:
                    self.sclk.append(cur)
                if pw:
                    self.power.append(int(open(pw[0]).read()) / 1e6)
            except Exception:
                pass
            self._stop.wait(0.005)

    def __enter__(self):
        import threading
        if self.dev:
            self._t = threading.Thread(target=self._run, daemon=True)
            self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._t:
            self._t.join()

    def summary(self):
        if not self.sclk:
            return None
        out = {"sclk_mhz": {"min": min(self.sclk), "median": statistics.median(self.sclk), "max": max(self.sclk),
                            "samples": len(self.sclk)}}
        if self.power:
            out["board_power_w"] = {"median": round(statistics.median(self.power), 1),
                                    "max": round(max(self.power), 1)}
        return out


def device_info(torch):
    """GPU identity and clock levels (sysfs pp_dpm tables), for the record."""
    pr = torch.cuda.get_device_properties(0)
    info = {"name": pr.name, "arch": pr.gcnArchName, "compute_units": pr.multi_processor_count,
            "memory_gib": round(pr.total_memory / 2 ** 30, 1)}
    d = _drm_device_dir(torch)
    try:
        if d:
            info["sclk_levels_mhz"] = _dpm_levels(os.path.join(d, "pp_dpm_sclk"))[0]
            mlev, mcur = _dpm_levels(os.path.join(d, "pp_dpm_mclk"))
            info["mclk_mhz"] = mcur if mcur is not None else (max(mlev) if mlev else None)
    except Exception:
        pass
    return info


def steady(torch, fn, ms=60.0):
    """Calls fn back to back for about `ms` of wall time so the timing that
    follows sees the steady-state shader clock: from idle the clock takes
    tens of milliseconds to ramp (the config-2 prefill measures 52-54 us
    cold, 45 us after 50 ms of calls)."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_graph(torch, g, reps):
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps  # ms


# ------------------------------------------------------------- config 5 ----
def build_config5(torch, aila_amd, steps, warmup):
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xA11A + 4)
    # KV capacity rounded up to a multiple of 1024 rows, as a serving engine
    # sizes it (block-aligned): a head stride aligned to 512 KiB keeps the
    # split-K decode's streams aligned (an odd row count costs ~7%).
    max_seq = (L5 + warmup + steps + 8 + 1023) // 1024 * 1024
    kc, vc = [], []
    for _ in range(N_GQA):
        k = torch.empty((B5, GQA_HKV, max_seq, GQA_D), dtype=torch.bfloat16, device=dev)
        v = torch.empty_like(k)
        k.normal_(generator=gen)
        v.normal_(generator=gen)
        kc.append(k)
        vc.append(v)
    states = [torch.empty((B5, DN_HV, DN_D, DN_D), dtype=torch.float32, device=dev).normal_(0, 0.02, generator=gen)
              for _ in range(N_LAYERS - N_GQA)]
    bf = dict(dtype=torch.bfloat16, device=dev)
    pool = []
    for _ in range(NPOOL):
        layers = []
        for layer in range(N_LAYERS):
            if layer % 4 == 3:
                layers.append(dict(q=torch.randn((B5, GQA_HQ, GQA_D), generator=gen, **bf),
                                   k=torch.randn((B5, GQA_HKV, GQA_D), generator=gen, **bf),
                                   v=torch.randn((B5, GQA_HKV, GQA_D), generator=gen, **bf)))
            else:
                layers.append(dict(q=torch.randn((B5, DN_HK, DN_D), generator=gen, **bf),
                                   k=torch.randn((B5, DN_HK, DN_D), generator=gen, **bf),
                                   v=torch.randn((B5, DN_HV, DN_D), generator=gen, **bf),
                                   a=torch.randn((B5, DN_HV), generator=gen, **bf),
                                   b=torch.randn((B5, DN_HV), generator=gen, **bf)))
        pool.append(layers)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B5, GQA_HQ, GQA_D), dtype=torch.uint8, device=dev)
    gqa_out = torch.empty((B5, GQA_HQ, GQA_D), **bf)
    dn_out = torch.empty((B5, DN_HV, DN_D), **bf)
    # device-side lengths: positions = row written this step (rows attended:
    # positions + 1)
    positions = torch.full((B5,), L5, dtype=torch.int32, device=dev)
    return dict(kc=kc, vc=vc, states=states, pool=pool, ws=ws, gqa_out=gqa_out, dn_out=dn_out,
                positions=positions, max_seq=max_seq)


def step5(aila_amd, W, p):
    """One decode token through the 32-layer stack (activation set p)."""
    gi = di = 0
    for layer in range(N_LAYERS):
        x = W["pool"][p][layer]
        if layer % 4 == 3:
            aila_amd.gqa_decode_append(x["q"], x["k"], x["v"], W["kc"][gi], W["vc"][gi], W["max_seq"] - 1,
                                       out=W["gqa_out"], workspace=W["ws"], positions=W["positions"])
            gi += 1
        else:
            aila_amd.deltanet_decode(x["q"], x["k"], x["v"], x["a"], x["b"], W["states"][di],
                                     out=W["dn_out"])
            di += 1
    W["positions"].add_(1)


def bench_config5(torch, aila_amd, steps, warmup, sampler=None):
    W = build_config5(torch, aila_amd, steps, warmup)
    graphs = []
    # capture NPOOL graphs, one per activation set; capture does not execute,
    # so lengths are unchanged by it.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step5(aila_amd, W, 0)     # warm the launch path once (eager)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    W["positions"].fill_(L5)
    for p in range(NPOOL):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step5(aila_amd, W, p)
        graphs.append(g)
    torch.cuda.synchronize()
    for i in range(warmup):
        graphs[i % NPOOL].replay()
    torch.cuda.synchronize()
    L_first = int(W["positions"][0].item()) + 1
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    import contextlib
    with sampler if sampler is not None else contextlib.nullcontext():
        t0 = time.perf_counter()
        s.record()
        for i in range(steps):
            graphs[(warmup + i) % NPOOL].replay()
        e.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms = s.elapsed_time(e) / steps
    # algorithmic bytes per step, averaged over the timed lengths
    L_mean = L_first + (steps - 1) / 2.0
    gqa_b = gqa_bytes(B5, GQA_HQ, GQA_HKV, GQA_D, L_mean) + 2 * B5 * GQA_HKV * GQA_D * 2 * 2
    dn_b = deltanet_bytes(B5, DN_HK, DN_HV, DN_D, DN_D)
    step_bytes = N_GQA * gqa_b + (N_LAYERS - N_GQA) * dn_b
    return dict(ms=ms, wall=wall, step_bytes=step_bytes, gqa_step_bytes=N_GQA * gqa_b,
                dn_step_bytes=(N_LAYERS - N_GQA) * dn_b, L_first=L_first, W=W)


def bench_config5_full_layers(torch, aila_amd, W, steps, warmup):
    """The config-5 step as the hybrid backend runs each layer
    (Qwen35HybridTextBackend.cpp:2109-2180 and :975-1166): every GQA layer is
    one launch of QK-norm + partial RoPE (rotary 64) + K/V append + split-K
    decode + the sigmoid(gate) epilogue from the packed q|gate projection
    (gqa_decode_prepare_append, packed_gate=2); every DeltaNet layer is the
    whole layer from the fused [qkv | z | a | b] row: conv1d ring + SiLU, L2
    norms, the recurrence and RMSNorm(o) * w * SiLU(z) (deltanet_layer_decode,
    one workgroup per value head). Same caches and states as the headline
    step; the conv ring heads and positions advance inside the graph."""
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xA11A + 9)
    bf = dict(dtype=torch.bfloat16, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    d, Hk, Hv = DN_D, DN_HK, DN_HV
    ch = 2 * Hk * d + Hv * d
    row = ch + Hv * d + 2 * Hv
    n_dn = N_LAYERS - N_GQA
    conv_w = [torch.randn((ch, 4), generator=gen, **bf) * 0.5 for _ in range(n_dn)]
    rings = [torch.empty((B5, 3, ch), **f32).normal_(generator=gen) for _ in range(n_dn)]
    norm_w = [1.0 + 0.1 * torch.randn(d, generator=gen, **f32) for _ in range(n_dn)]
    arrivals = [torch.zeros((B5 * Hk,), dtype=torch.int32, device=dev) for _ in range(n_dn)]
    qn_w = [torch.randn(GQA_D, generator=gen, **bf) for _ in range(N_GQA)]
    kn_w = [torch.randn(GQA_D, generator=gen, **bf) for _ in range(N_GQA)]
    pool = []
    for _ in range(NPOOL):
        layers = []
        for layer in range(N_LAYERS):
            if layer % 4 == 3:
                layers.append(dict(q=torch.randn((B5, GQA_HQ, 2 * GQA_D), generator=gen, **bf),
                                   k=torch.randn((B5, GQA_HKV, GQA_D), generator=gen, **bf),
                                   v=torch.randn((B5, GQA_HKV, GQA_D), generator=gen, **bf)))
            else:
                layers.append(dict(row=torch.randn((B5, row), generator=gen, **bf)))
        pool.append(layers)
    gqa_out = torch.empty((B5, GQA_HQ, GQA_D), **bf)
    dn_out = torch.empty((B5, Hv * d), **bf)
    heads = torch.zeros((B5,), dtype=torch.int32, device=dev)
    positions = torch.full((B5,), L5, dtype=torch.int32, device=dev)

    def step(p):
        gi = di = 0
        for layer in range(N_LAYERS):
            x = pool[p][layer]
            if layer % 4 == 3:
                aila_amd.gqa_decode_prepare_append(x["q"], x["k"], x["v"], W["kc"][gi], W["vc"][gi],
                                                   W["max_seq"] - 1, q_norm_w=qn_w[gi], k_norm_w=kn_w[gi],
                                                   rotary_dim=64, theta=1e7, packed_gate=True, apply_gate=True,
                                                   out=gqa_out, workspace=W["ws"], positions=positions)
                gi += 1
            else:
                r = x["row"]
                aila_amd.deltanet_layer_decode(r[:, :ch], r[:, ch:ch + Hv * d], r[:, ch + Hv * d:ch + Hv * d + Hv],
                                               r[:, ch + Hv * d + Hv:], conv_w[di], rings[di], 0, norm_w[di],
                                               W["states"][di], Hk, out=dn_out, conv_heads=heads,
                                               arrivals=arrivals[di])
                di += 1
        positions.add_(1)
        heads.add_(1).remainder_(3)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    positions.fill_(L5)
    graphs = []
    for p in range(NPOOL):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(p)
        graphs.append(g)
    torch.cuda.synchronize()
    for i in range(warmup):
        graphs[i % NPOOL].replay()
    torch.cuda.synchronize()
    L_first = int(positions[0].item()) + 1
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(steps):
        graphs[(warmup + i) % NPOOL].replay()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps
    L_mean = L_first + (steps - 1) / 2.0
    # GQA layer: K/V rows read, packed q|gate in, k/v in, k/v rows written, out
    gqa_b = (2 * B5 * GQA_HKV * L_mean * GQA_D * 2 + B5 * GQA_HQ * 2 * GQA_D * 2 + 2 * B5 * GQA_HKV * GQA_D * 2 * 2
             + B5 * GQA_HQ * GQA_D * 2)
    dn_b = deltanet_layer_bytes(B5, Hk, Hv, d)
    step_bytes = N_GQA * gqa_b + n_dn * dn_b
    del graphs, pool, rings
    return {"config": ("config-5 stack, each layer as the backend runs it: GQA = norm + RoPE(64) + append + "
                       "split-K decode + sigmoid(gate) in one launch; DeltaNet = conv ring + SiLU + norms + "
                       "recurrence + gated RMSNorm in one launch"),
            "ms_per_step": round(ms, 4), "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "step_bytes": int(step_bytes), "context": L_first, "steps": steps}


def roofline_gqa(torch, aila_amd, W, reps=64):
    """Dominant kernel: one GQA decode launch (split + merge dispatch) on a
    config-5 layer at L = 32768, timed with HIP events around a batch of
    back-to-back launches on the stream the kernels run on (torch's current
    stream)."""
    L = L5
    lens = torch.full((B5,), L, dtype=torch.int32, device="cuda")
    x = W["pool"][0][3]
    fn = lambda: aila_amd.gqa_decode(x["q"], W["kc"][0], W["vc"][0], L, out=W["gqa_out"],
                                     workspace=W["ws"], seq_lens=lens)
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    # One event pair around `reps` back-to-back launches (an event pair per
    # launch adds its own gap to every measured interval). A spin kernel
    # queued first keeps the device busy while the host enqueues, so the
    # interval holds device work only.
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2.4e9 * 0.02))   # ~20 ms at 2.4 GHz
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    avg_ms = s.elapsed_time(e) / reps
    byts = gqa_bytes(B5, GQA_HQ, GQA_HKV, GQA_D, L)
    achieved = byts / (avg_ms * 1e-3) / 1e9
    # HBM bytes per launch from the committed counter runs, used only while
    # the kernel source they were measured on is unchanged (source stamp).
    traffic, note = None, "no counter profile"
    tpath = os.path.join(ROOT, "profiles", "gqa_decode_config5_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            prof = json.load(f)
        if prof.get("source_sha16") == decode_source_stamp():
            traffic = prof.get("hbm_bytes_per_launch")
            note = "rocprofv3 FETCH_SIZE + WRITE_SIZE of this kernel source, calibrated on a 1 GiB copy"
        else:
            note = "counter profile is stale (kernel source changed since it was measured)"
    out = {"kernel": "gqa_decode_split_kernel<256,4> + merge", "bound": "hbm",
           "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": note,
           "algorithmic_bytes": byts, "avg_launch_us": round(avg_ms * 1e3, 2)}
    ach = achievable_read(torch, W["kc"][0], W["vc"][0], L, reps)
    if ach is not None:
        out["achievable"] = dict(ach, frac_of_achievable=round(achieved / ach["read_gbs"], 4))
    return out


def achievable_read(torch, kc, vc, L, reps):
    """The streaming-read probe (aila_amd/libaila_probe.so) over the same
    K/V rows the decode launch reads, in as many workgroups (one round of
    resident workgroups: 16 splits per sequence and KV head at config 5),
    timed like the decode. None if the probe library is absent."""
    import ctypes
    path = os.path.join(ROOT, "aila_amd", "libaila_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.aila_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_long, ctypes.c_long, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_void_p]
    lib.aila_probe_stream_read.restype = ctypes.c_int
    B, Hkv, max_seq, D = kc.shape
    nsplit = max(1, 512 // (B * Hkv))
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def fn():
        rc = lib.aila_probe_stream_read(kc.data_ptr(), vc.data_ptr(), B, Hkv, max_seq, L, D, nsplit,
                                        sink.data_ptr(), stream)
        if rc != 0:
            raise RuntimeError(f"aila_probe_stream_read: hipError {rc}")
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2.4e9 * 0.02))
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    avg_ms = s.elapsed_time(e) / reps
    byts = 2 * B * Hkv * L * D * 2
    return {"read_gbs": round(byts / (avg_ms * 1e-3) / 1e9, 1), "read_bytes": byts,
            "avg_launch_us": round(avg_ms * 1e3, 2),
            "probe": f"streaming read of the same K/V rows, {nsplit * Hkv * B} workgroups, 16-byte nontemporal loads"}


def achievable_rw_us(torch, states, per_graph=16, reps=32, blocks=(256, 512, 1024, 2048)):
    """In-place read + write probe (aila_amd/libaila_probe.so) over the given
    fp32 states, one launch per state in graph replay as the decode steps are
    timed: microseconds per launch at the best of the grid sizes tried, the
    floor a step that reads and writes its state once reaches on this box.
    None if the probe library is absent."""
    import ctypes
    path = os.path.join(ROOT, "aila_amd", "libaila_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.aila_probe_stream_rw.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    lib.aila_probe_stream_rw.restype = ctypes.c_int
    seq = [states[i % len(states)] for i in range(max(per_graph, len(states)))]
    stream = torch.cuda.current_stream().cuda_stream

    def launch(t, nb, st_ptr):
        rc = lib.aila_probe_stream_rw(t.data_ptr(), t.numel() * t.element_size(), nb, st_ptr)
        if rc != 0:
            raise RuntimeError(f"aila_probe_stream_rw: hipError {rc}")
    best = None
    for nb in blocks:
        for t in seq:
            launch(t, nb, stream)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            cap = torch.cuda.current_stream().cuda_stream
            for t in seq:
                launch(t, nb, cap)
        gr.replay()
        us = time_graph(torch, gr, reps) * 1e3 / len(seq)
        best = us if best is None else min(best, us)
    return best


def decode_source_stamp():
    """First 16 hex digits of the SHA-256 of the GQA decode kernel sources."""
    import hashlib
    h = hashlib.sha256()
    for name in ("gqa_decode.hip", "common.hpp"):
        with open(os.path.join(ROOT, "aila_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def write_traffic(fetch_csv, write_csv):
    """Builds profiles/gqa_decode_config5_traffic.json from the two
    `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of
    `bench.py --profile-kernel gqa_decode` (their run_counter_collection.csv):
    medians per kernel, scaled by what each counter reads for the 1 GiB
    device copy of the same run (1 GiB read, 1 GiB written)."""
    import csv

    def medians(path):
        vals = {}
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return {k: statistics.median(v) for k, v in vals.items()}

    def pick(m, key):
        names = [k for k in m if key in k]
        if not names:
            raise SystemExit(f"no dispatch of a kernel named *{key}* in the counter file")
        return max(names, key=lambda k: m[k])

    F, Wr = medians(fetch_csv), medians(write_csv)
    gib_kib = float(1 << 20)
    cf, cw = pick(F, "copy"), pick(Wr, "copy")
    fs, ws_ = gib_kib / F[cf], gib_kib / Wr[cw]
    sk, mk = pick(F, "gqa_decode_split_kernel"), pick(F, "gqa_decode_merge_kernel")
    fetch = {"split": F[sk], "merge": F[mk]}
    write = {"split": Wr[pick(Wr, "gqa_decode_split_kernel")], "merge": Wr[pick(Wr, "gqa_decode_merge_kernel")]}
    hbm = int(round(1024 * (fs * (fetch["split"] + fetch["merge"]) + ws_ * (write["split"] + write["merge"]))))
    out = {"kernel": "gqa_decode_split_kernel<256,4> + gqa_decode_merge_kernel<256>",
           "workload": "config 5 GQA layer: B=8 Hq=16 Hkv=4 D=256 L=32768",
           "fetch_kib": {k: round(v, 1) for k, v in fetch.items()},
           "write_kib": {k: round(v, 1) for k, v in write.items()},
           "fetch_scale": round(fs, 4), "write_scale": round(ws_, 4),
           "hbm_bytes_per_launch": hbm,
           "algorithmic_bytes_per_launch": gqa_bytes(B5, GQA_HQ, GQA_HKV, GQA_D, L5),
           "source_sha16": decode_source_stamp(),
           "source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE -- python3 bench.py --profile-kernel gqa_decode"}
    with open(os.path.join(ROOT, "profiles", "gqa_decode_config5_traffic.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out))


def profile_kernel(torch, aila_amd, reps=20):
    """Dominant kernel alone (one config-5 GQA layer, B=8, L=32768) plus a
    plain 1 GiB device-to-device copy used to calibrate the HBM byte
    counters (FETCH_SIZE / WRITE_SIZE) against a known traffic."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(0xA11A + 4)
    bf = dict(dtype=torch.bfloat16, device=dev)
    kc = torch.empty((B5, GQA_HKV, L5, GQA_D), **bf).normal_(generator=g)
    vc = torch.empty_like(kc).normal_(generator=g)
    q = torch.randn((B5, GQA_HQ, GQA_D), generator=g, **bf)
    out = torch.empty_like(q)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B5, GQA_HQ, GQA_D), dtype=torch.uint8, device=dev)
    src = torch.empty(1 << 29, **bf).normal_(generator=g)   # 1 GiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        aila_amd.gqa_decode(q, kc, vc, L5, out=out, workspace=ws)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[profile] gqa_decode x{reps} (algorithmic {gqa_bytes(B5, GQA_HQ, GQA_HKV, GQA_D, L5)} B/launch), "
        f"copy x{reps} ({2 * src.numel() * 2} B/launch: 1 GiB read + 1 GiB write)")


# ------------------------------------------------------------ sub-metrics --
def sub_prefill(torch, aila_amd, reps=100):
    S, Hq, Hkv, D = 2048, 32, 8, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 1)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    q = torch.randn((S, Hq * D), generator=g, **bf)
    k = torch.randn((S, Hkv * D), generator=g, **bf)
    v = torch.randn((S, Hkv * D), generator=g, **bf)
    # config 2's inputs: per-head QK RMS-norm (weight 1) and NeoX RoPE
    # (theta 1e6, positions 0..S-1) on q and k, prepared outside the timing
    aila_amd.head_rms_norm(q.view(S, Hq, D), eps=1e-6)
    aila_amd.head_rms_norm(k.view(S, Hkv, D), eps=1e-6)
    aila_amd.apply_rope(q.view(S, Hq, D), k.view(S, Hkv, D), start_pos=0, rotary_dim=D, theta=1e6)
    out = torch.empty_like(q)
    kc = torch.empty((Hkv, S, D), **bf)
    vc = torch.empty_like(kc)
    fn = lambda: aila_amd.gqa_prefill(q, k, v, Hq, Hkv, out=out, k_cache=kc, v_cache=vc)
    steady(torch, fn)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) / reps * 1e3
    flops = 4 * D * Hq * S * (S + 1) / 2
    res = {"config": "2: S=2048 Hq=32 Hkv=8 D=128 causal (QK-normed, RoPE'd inputs) + cache write", "us": round(us, 2),
           "tflops": round(flops / us / 1e6, 1), "frac_of_bf16_peak": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4)}
    ach = achievable_mfma(torch)
    if ach is not None:
        res["achievable_mfma_tflops"] = ach
        res["frac_of_achievable"] = round(flops / us / 1e6 / ach, 4)
    return res


def achievable_mfma(torch, blocks=1024, iters=8192):
    """Dense bf16 MFMA rate the chip sustains (aila_amd/libaila_probe.so:
    independent v_mfma_f32_16x16x32_bf16 streams on every SIMD), TFLOP/s,
    or None if the probe library is absent."""
    import ctypes
    path = os.path.join(ROOT, "aila_amd", "libaila_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.aila_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.aila_probe_mfma.restype = ctypes.c_int
    sink = torch.zeros(1, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def fn():
        rc = lib.aila_probe_mfma(blocks, iters, sink.data_ptr(), stream)
        if rc != 0:
            raise RuntimeError(f"aila_probe_mfma: hipError {rc}")
    fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(3):
        fn()
    e.record()
    torch.cuda.synchronize()
    sec = s.elapsed_time(e) / 3 * 1e-3
    return round(blocks * 4 * iters * 16 * 16384 / sec / 1e12, 1)


def sub_prefill_cached(torch, aila_amd, reps=20):
    """Multi-turn prefill over a cached prefix (next row 3 of the path):
    a Qwen3.5 full-attention layer (16 q / 4 kv heads, D=256) appends a
    512-token turn to a 4096-token cache and attends it causally, then the
    gated-attention epilogue out *= sigmoid(gate)."""
    S, start, Hq, Hkv, D = 512, 4096, 16, 4, 256
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 6)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    max_seq = start + S
    kc = torch.randn((Hkv, max_seq, D), generator=g, **bf)
    vc = torch.randn((Hkv, max_seq, D), generator=g, **bf)
    q = torch.randn((S, Hq * D), generator=g, **bf)
    gate = torch.randn((S, Hq * D), generator=g, **bf)
    out = torch.empty_like(q)

    ws = torch.empty(max(aila_amd.gqa_prefill_cached_workspace_size(S, start, Hq, Hkv, D), 16), dtype=torch.uint8,
                     device="cuda")

    def timed(fn):
        # HIP-graph replay of `reps` calls: the kernels' time, not the host's
        steady(torch, fn)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(reps):
                fn()
        gr.replay()
        return time_graph(torch, gr, 3) * 1e3 / reps

    us_split = timed(lambda: aila_amd.gqa_prefill_cached(q, kc, vc, start, Hq, out=out, workspace=ws))
    us_whole = timed(lambda: aila_amd.gqa_prefill_cached(q, kc, vc, start, Hq, out=out))
    us_gate = timed(lambda: aila_amd.sigmoid_mul(out, gate, out=out))
    flops = 4 * D * Hq * (S * start + S * (S + 1) / 2)
    gate_bytes = 3 * S * Hq * D * 2
    return {"config": f"prefill over a cached prefix: S={S} new tokens after {start}, Hq={Hq} Hkv={Hkv} D={D}; "
                      "then out *= sigmoid(gate)",
            "attn_us": round(us_split, 2), "attn_tflops": round(flops / us_split / 1e6, 1),
            "attn_frac_of_bf16_peak": round(flops / us_split / 1e6 / BF16_PEAK_TFLOPS, 4),
            "key_split_workspace_bytes": int(ws.numel()) if ws.numel() > 16 else 0,
            "attn_no_split_us": round(us_whole, 2),
            "sigmoid_mul_us": round(us_gate, 2), "sigmoid_mul_GBps": round(gate_bytes / us_gate / 1e3, 1)}


def sub_deltanet_decode(torch, aila_amd, steps=2048, per_graph=16):
    B, H, d = 32, 16, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 2)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    st = torch.empty((B, H, d, d), dtype=torch.float32, device="cuda").normal_(0, 0.02, generator=g)
    xs = [dict(q=torch.randn((B, H, d), generator=g, **bf), k=torch.randn((B, H, d), generator=g, **bf),
               v=torch.randn((B, H, d), generator=g, **bf), a=torch.randn((B, H), generator=g, **bf),
               b=torch.randn((B, H), generator=g, **bf)) for _ in range(per_graph)]
    out = torch.empty((B, H, d), **bf)
    for x in xs:
        aila_amd.deltanet_decode(x["q"], x["k"], x["v"], x["a"], x["b"], st, out=out)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for x in xs:
            aila_amd.deltanet_decode(x["q"], x["k"], x["v"], x["a"], x["b"], st, out=out)
    gr.replay()
    ms = time_graph(torch, gr, steps // per_graph)
    us = ms * 1e3 / per_graph
    byts = deltanet_bytes(B, H, H, d, d)
    bound_us = byts / (HBM_PEAK_GBS * 1e3)
    # Sequential steps of one recurrence keep its 67 MB state in the 256 MB
    # Infinity Cache. The same step with the state evicted: eight states in
    # rotation, each touched again only after 470 MB of other states' traffic.
    nst = 8
    sts = [torch.empty_like(st).normal_(0, 0.02, generator=g) for _ in range(nst)]
    for s_ in sts:
        aila_amd.deltanet_decode(xs[0]["q"], xs[0]["k"], xs[0]["v"], xs[0]["a"], xs[0]["b"], s_, out=out)
    torch.cuda.synchronize()
    grc = torch.cuda.CUDAGraph()
    with torch.cuda.graph(grc):
        for i, s_ in enumerate(sts):
            x = xs[i % per_graph]
            aila_amd.deltanet_decode(x["q"], x["k"], x["v"], x["a"], x["b"], s_, out=out)
    grc.replay()
    us_cold = time_graph(torch, grc, max(steps // nst // 4, 8)) * 1e3 / nst
    res = {"config": "3: B=32 H=16 dk=dv=128, 2048 sequential steps", "us_per_step": round(us, 3),
           "GBps": round(byts / us / 1e3, 1), "x_of_state_traffic_bound": round(us / bound_us, 3),
           "state_evicted_us_per_step": round(us_cold, 3),
           "state_evicted_x_of_bound": round(us_cold / bound_us, 3)}
    ach, ach_cold = achievable_rw_us(torch, [st]), achievable_rw_us(torch, sts)
    del sts
    if ach is not None:
        res["achievable"] = {"probe": "in-place read + write of the same state(s), 16-byte nontemporal, graph replay, best of 256-2048 workgroups",
                             "rw_us": round(ach, 3), "x_of_achievable": round(us / ach, 3),
                             "state_evicted_rw_us": round(ach_cold, 3),
                             "state_evicted_x_of_achievable": round(us_cold / ach_cold, 3)}
    return res


def sub_deltanet_layer_decode(torch, aila_amd, steps=512, per_graph=16):
    """Full layer decode (conv ring + SiLU + norms + recurrence + gated RMSNorm)
    at the config-5 DeltaNet layer shape, next to the recurrence-only kernel
    on the same state."""
    B, Hk, Hv, d = B5, DN_HK, DN_HV, DN_D
    ch = 2 * Hk * d + Hv * d
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 5)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    f32 = dict(dtype=torch.float32, device="cuda")
    st = torch.empty((B, Hv, d, d), **f32).normal_(0, 0.02, generator=g)
    cs = torch.empty((B, 3, ch), **f32).normal_(generator=g)
    w = torch.randn((ch, 4), generator=g, **bf)
    nw = torch.ones(d, **f32)
    xs = [dict(qkv=torch.randn((B, ch), generator=g, **bf), z=torch.randn((B, Hv * d), generator=g, **bf),
               a=torch.randn((B, Hv), generator=g, **bf), b=torch.randn((B, Hv), generator=g, **bf))
          for _ in range(per_graph)]
    out = torch.empty((B, Hv * d), **bf)
    heads = torch.zeros((B,), dtype=torch.int32, device="cuda")
    # arrival counts (zeroed once, left zero by every call): one workgroup per
    # value head
    arr = torch.zeros((B * Hk,), dtype=torch.int32, device="cuda")
    fn = lambda x: aila_amd.deltanet_layer_decode(x["qkv"], x["z"], x["a"], x["b"], w, cs, 0, nw, st, Hk,
                                                  out=out, conv_heads=heads, arrivals=arr)
    for x in xs:
        fn(x)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for x in xs:
            fn(x)
    gr.replay()
    us = time_graph(torch, gr, steps // per_graph) * 1e3 / per_graph
    byts = deltanet_layer_bytes(B, Hk, Hv, d)
    # the recurrence-only kernel on the same shape
    q = [torch.randn((B, Hk, d), generator=g, **bf) for _ in range(2)]
    v = torch.randn((B, Hv, d), generator=g, **bf)
    o2 = torch.empty((B, Hv, d), **bf)
    gr2 = torch.cuda.CUDAGraph()
    aila_amd.deltanet_decode(q[0], q[1], v, xs[0]["a"], xs[0]["b"], st, out=o2)
    torch.cuda.synchronize()
    with torch.cuda.graph(gr2):
        for _ in range(per_graph):
            aila_amd.deltanet_decode(q[0], q[1], v, xs[0]["a"], xs[0]["b"], st, out=o2)
    gr2.replay()
    us2 = time_graph(torch, gr2, steps // per_graph) * 1e3 / per_graph
    # As in the config-5 stack: 24 layers, each with its own state (403 MB
    # in all), so every step finds its state evicted from the caches.
    nl = N_LAYERS - N_GQA
    sts = [torch.empty_like(st).normal_(0, 0.02, generator=g) for _ in range(nl)]
    css = [torch.empty_like(cs).normal_(generator=g) for _ in range(nl)]
    gr3 = torch.cuda.CUDAGraph()
    gr4 = torch.cuda.CUDAGraph()
    x0 = xs[0]
    with torch.cuda.graph(gr3):
        for i in range(nl):
            aila_amd.deltanet_layer_decode(x0["qkv"], x0["z"], x0["a"], x0["b"], w, css[i], 0, nw, sts[i], Hk,
                                           out=out, conv_heads=heads, arrivals=arr)
    with torch.cuda.graph(gr4):
        for i in range(nl):
            aila_amd.deltanet_decode(q[0], q[1], v, x0["a"], x0["b"], sts[i], out=o2)
    gr3.replay()
    gr4.replay()
    us3 = time_graph(torch, gr3, max(steps // nl, 8)) * 1e3 / nl
    us4 = time_graph(torch, gr4, max(steps // nl, 8)) * 1e3 / nl
    ach, ach_cold = achievable_rw_us(torch, [st]), achievable_rw_us(torch, sts)
    del sts, css
    rb = deltanet_bytes(B, Hk, Hv, d, d)
    res = {"config": f"layer decode B={B} Hk={Hk} Hv={Hv} d={d} (config-5 DeltaNet layer)",
           "us_per_step": round(us, 3), "GBps": round(byts / us / 1e3, 1),
           "x_of_bound": round(us / (byts / (HBM_PEAK_GBS * 1e3)), 3),
           "recurrence_only_us": round(us2, 3),
           "recurrence_only_x_of_bound": round(us2 / (rb / (HBM_PEAK_GBS * 1e3)), 3),
           "state_evicted_us": round(us3, 3),
           "state_evicted_x_of_bound": round(us3 / (byts / (HBM_PEAK_GBS * 1e3)), 3),
           "state_evicted_recurrence_only_us": round(us4, 3),
           "state_evicted_recurrence_only_x_of_bound": round(us4 / (rb / (HBM_PEAK_GBS * 1e3)), 3),
           "state_evicted_note": "24 states in rotation, one per DeltaNet layer of the config-5 stack"}
    if ach is not None:
        res["achievable"] = {"probe": "in-place read + write of the same state(s), 16-byte nontemporal, graph replay, best of 256-2048 workgroups",
                             "rw_us": round(ach, 3), "x_of_achievable": round(us / ach, 3),
                             "recurrence_only_x_of_achievable": round(us2 / ach, 3),
                             "state_evicted_rw_us": round(ach_cold, 3),
                             "state_evicted_x_of_achievable": round(us3 / ach_cold, 3),
                             "state_evicted_recurrence_only_x_of_achievable": round(us4 / ach_cold, 3)}
    return res


def sub_deltanet_prefill(torch, aila_amd, reps=40):
    B, T, Hk, Hv, d = 1, 4096, 16, 32, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 3)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    q = torch.randn((B, T, Hk, d), generator=g, **bf)
    k = torch.randn((B, T, Hk, d), generator=g, **bf)
    v = torch.randn((B, T, Hv, d), generator=g, **bf)
    a = torch.randn((B, T, Hv), generator=g, **bf)
    b = torch.randn((B, T, Hv), generator=g, **bf)
    st = torch.zeros((B, Hv, d, d), dtype=torch.float32, device="cuda")
    out = torch.empty((B, T, Hv, d), **bf)
    ws = torch.empty(aila_amd.deltanet_prefill_workspace_size(B, T, Hv, d, d), dtype=torch.uint8, device="cuda")
    fn = lambda: aila_amd.deltanet_prefill(q, k, v, a, b, st, out=out, workspace=ws)
    steady(torch, fn)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) / reps * 1e3
    byts = 103.8e6
    flops = 23.98e9
    frac = max(byts / (HBM_PEAK_GBS * 1e9), flops / (BF16_PEAK_TFLOPS * 1e12)) / (us * 1e-6)
    return {"config": "4: T=4096 C=64 Hk=16 Hv=32 dk=dv=128", "us": round(us, 1),
            "tok_per_s": round(T / (us * 1e-6)), "roofline_frac": round(frac, 4)}


def sub_fused_prep_decode(torch, aila_amd, per_graph=8, reps=8):
    """One config-5 GQA layer step (B=8, Hq=16, Hkv=4, D=256, rotary 64,
    packed q|gate, context 32768): the one-launch prep + append + decode
    against the two launches decode_prepare_qkv + gqa_decode_append."""
    B, Hq, Hkv, D, rot, L = B5, GQA_HQ, GQA_HKV, GQA_D, 64, 32768
    max_seq = L + 1024
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 7)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    kc = torch.empty((B, Hkv, max_seq, D), **bf).normal_(generator=g)
    vc = torch.empty_like(kc).normal_(generator=g)
    qg = torch.randn((B, Hq, 2 * D), generator=g, **bf)
    k = torch.randn((B, Hkv, D), generator=g, **bf)
    v = torch.randn((B, Hkv, D), generator=g, **bf)
    wq, wk = torch.randn(D, generator=g, **bf), torch.randn(D, generator=g, **bf)
    pos = torch.full((B,), L, dtype=torch.int32, device="cuda")
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out, go, qo = (torch.empty((B, Hq, D), **bf) for _ in range(3))
    kk = torch.empty_like(k)

    def fused():
        aila_amd.gqa_decode_prepare_append(qg, k, v, kc, vc, L, q_norm_w=wq, k_norm_w=wk, rotary_dim=rot,
                                           theta=1e7, packed_gate=True, out=out, gate_out=go, workspace=ws,
                                           positions=pos)

    def fused_gated():
        aila_amd.gqa_decode_prepare_append(qg, k, v, kc, vc, L, q_norm_w=wq, k_norm_w=wk, rotary_dim=rot,
                                           theta=1e7, packed_gate=True, apply_gate=True, out=out, workspace=ws,
                                           positions=pos)

    def fused_then_gate():
        fused()
        aila_amd.sigmoid_mul(out, go, out=out)

    def two():
        kk.copy_(k)   # decode_prepare_qkv normalises and rotates k in place
        aila_amd.decode_prepare_qkv(qg, kk, v, wq, wk, None, None, positions=pos, rotary_dim=rot, theta=1e7,
                                    packed_gate=True, q_out=qo, gate_out=go)
        aila_amd.gqa_decode_append(qo, kk, v, kc, vc, L, out=out, workspace=ws, positions=pos)

    res = {}
    for name, fn in (("fused_us", fused), ("two_launch_us", two), ("fused_gated_us", fused_gated),
                     ("fused_then_sigmoid_mul_us", fused_then_gate)):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(per_graph):
                fn()
        gr.replay()
        res[name] = round(time_graph(torch, gr, reps) * 1e3 / per_graph, 2)
    del kc, vc
    res["config"] = "config-5 GQA layer step B=8 Hq=16 Hkv=4 D=256 L=32768, prep + append + decode"
    res["two_launch_note"] = "includes a 32 KiB device copy of k (the two-launch prep rotates k in place)"
    res["gated_note"] = ("fused_gated_us applies out *= sigmoid(gate) in the merge (apply_gate); "
                         "fused_then_sigmoid_mul_us is the same work as two launches")
    return res


def sub_decode_prep(torch, aila_amd, per_graph=32, reps=20):
    """QK-norm + partial RoPE + packed q|gate split + K/V append for one
    config-5 GQA layer (B=8, Hq=16, Hkv=4, D=256, rotary 64)."""
    B, Hq, Hkv, D, rot = B5, GQA_HQ, GQA_HKV, GQA_D, 64
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 6)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    qg = torch.randn((B, Hq, 2 * D), generator=g, **bf)
    k = torch.randn((B, Hkv, D), generator=g, **bf)
    v = torch.randn((B, Hkv, D), generator=g, **bf)
    wq, wk = torch.randn(D, generator=g, **bf), torch.randn(D, generator=g, **bf)
    kc = torch.empty((B, Hkv, 1024, D), **bf)
    vc = torch.empty_like(kc)
    qo, go = torch.empty((B, Hq, D), **bf), torch.empty((B, Hq, D), **bf)
    pos = torch.full((B,), 700, dtype=torch.int32, device="cuda")
    fn = lambda: aila_amd.decode_prepare_qkv(qg, k, v, wq, wk, kc, vc, positions=pos, rotary_dim=rot,
                                             theta=1e7, packed_gate=True, q_out=qo, gate_out=go)
    fn()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for _ in range(per_graph):
            fn()
    gr.replay()
    us = time_graph(torch, gr, reps) * 1e3 / per_graph
    byts = B * Hq * 2 * D * 2 + 2 * B * Hq * D * 2 + 2 * B * Hkv * D * 2 + 3 * B * Hkv * D * 2
    return {"config": f"decode prep B={B} Hq={Hq} Hkv={Hkv} D={D} rot={rot} packed q|gate",
            "us_per_call": round(us, 2), "GBps": round(byts / us / 1e3, 1)}


def sub_deltanet_layer_prefill(torch, aila_amd, reps=40):
    """Full layer prefill (conv ring + SiLU into hi/lo planes, chunked
    recurrence with the key/value residuals, RMSNorm*SiLU(z) gate) at the
    config-4 shape, from the backend's fused [qkv | z | a | b] rows."""
    B, T, Hk, Hv, d = 1, 4096, 16, 32, 128
    ch, zd = 2 * Hk * d + Hv * d, Hv * d
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 7)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    fused = torch.randn((B, T, ch + zd + 2 * Hv), generator=g, **bf)
    w = torch.randn((ch, 4), generator=g, **bf) * 0.5
    cs = torch.zeros((B, 3, ch), dtype=torch.float32, device="cuda")
    nw = torch.ones(d, dtype=torch.float32, device="cuda")
    st = torch.zeros((B, Hv, d, d), dtype=torch.float32, device="cuda")
    ws = torch.empty(aila_amd.deltanet_layer_prefill_workspace_size(B, T, Hk, Hv), dtype=torch.uint8, device="cuda")
    out = torch.empty((B, T, zd), **bf)
    fn = lambda: aila_amd.deltanet_layer_prefill(fused[..., :ch], fused[..., ch:ch + zd],
                                                 fused[..., ch + zd:ch + zd + Hv], fused[..., ch + zd + Hv:], w, cs, 0,
                                                 nw, st, Hk, out=out, workspace=ws)
    steady(torch, fn)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) / reps * 1e3
    return {"config": f"layer prefill T={T} Hk={Hk} Hv={Hv} d={d} (fused rows)", "us": round(us, 1),
            "tok_per_s": round(T / (us * 1e-6))}


def sub_paged_decode(torch, aila_amd, page_size=256, reps=32):
    """One config-5 GQA layer (B=8, Hq=16, Hkv=4, D=256, L=32768) over a
    paged cache (pages of page_size rows scattered in a shuffled pool) next
    to the same rows in the contiguous layout; HIP events around `reps`
    back-to-back launches each."""
    B, Hq, Hkv, D, L = B5, GQA_HQ, GQA_HKV, GQA_D, L5
    mp = L // page_size
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 8)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    pk = torch.empty((B * mp, Hkv, page_size, D), **bf).normal_(generator=g)
    pv = torch.empty_like(pk).normal_(generator=g)
    table = torch.randperm(B * mp, generator=torch.Generator().manual_seed(7)).to(torch.int32).view(B, mp).cuda()
    q = torch.randn((B, Hq, D), generator=g, **bf)
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    fn = lambda: aila_amd.gqa_decode_paged(q, pk, pv, table, lens, L, out=out, workspace=ws)
    res = {}
    for name, f in (("paged", fn),):
        for _ in range(3):
            f()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2.4e9 * 0.01))
        s.record()
        for _ in range(reps):
            f()
        e.record()
        torch.cuda.synchronize()
        res[name + "_us"] = round(s.elapsed_time(e) / reps * 1e3, 2)
    del pk, pv
    kc = torch.empty((B, Hkv, L, D), **bf).normal_(generator=g)
    vc = torch.empty_like(kc).normal_(generator=g)
    f = lambda: aila_amd.gqa_decode(q, kc, vc, L, out=out, workspace=ws, seq_lens=lens)
    for _ in range(3):
        f()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.4e9 * 0.01))
    s.record()
    for _ in range(reps):
        f()
    e.record()
    torch.cuda.synchronize()
    res["contiguous_us"] = round(s.elapsed_time(e) / reps * 1e3, 2)
    byts = gqa_bytes(B, Hq, Hkv, D, L)
    res["paged_GBps"] = round(byts / res["paged_us"] / 1e3, 1)
    res["contiguous_GBps"] = round(byts / res["contiguous_us"] / 1e3, 1)
    res["config"] = f"config-5 GQA layer B={B} L={L} over {page_size}-row pages (shuffled pool) vs contiguous"
    del kc, vc
    return res


def sub_decode_cfg1(torch, aila_amd, per_graph=32, reps=20):
    B, Hq, Hkv, D, L = 1, 16, 8, 128, 512
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    q = torch.randn((B, Hq, D), generator=g, **bf)
    kc = torch.randn((B, Hkv, L, D), generator=g, **bf)
    vc = torch.randn((B, Hkv, L, D), generator=g, **bf)
    ws = torch.empty(aila_amd.gqa_decode_workspace_size(B, Hq, D), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    aila_amd.gqa_decode(q, kc, vc, L, out=out, workspace=ws)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for _ in range(per_graph):
            aila_amd.gqa_decode(q, kc, vc, L, out=out, workspace=ws)
    gr.replay()
    us = time_graph(torch, gr, reps) * 1e3 / per_graph
    byts = gqa_bytes(B, Hq, Hkv, D, L)
    return {"config": "1: B=1 Hq=16 Hkv=8 D=128 L=512", "us_per_call": round(us, 2),
            "GBps": round(byts / us / 1e3, 1)}


def sub_single_sequence(torch, aila_amd, per_graph=8, reps=20):
    """The reference engine runs one sequence at a time: the path's kernels
    at batch 1 and for short prompts (the Qwen3.5-4B and Qwen3-4B shapes),
    each timed by HIP-graph replay. Not a config of the benchmark; reported
    beside it."""
    g = torch.Generator(device="cuda")
    g.manual_seed(0xA11A + 6)
    bf = dict(dtype=torch.bfloat16, device="cuda")

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(per_graph):
                fn()
        gr.replay()
        return round(time_graph(torch, gr, reps) * 1e3 / per_graph, 2)

    res = {"note": "batch 1 and short prompts (the reference's single-sequence use); us per call, graph replay"}
    for L in (8192, 32768):   # Qwen3.5 full-attention layer decode
        Hq, Hkv, D = GQA_HQ, GQA_HKV, GQA_D
        q = torch.randn((1, Hq, D), generator=g, **bf)
        kc = torch.randn((1, Hkv, L, D), generator=g, **bf)
        vc = torch.randn_like(kc)
        ws = torch.empty(aila_amd.gqa_decode_workspace_size(1, Hq, D), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        us = timed(lambda: aila_amd.gqa_decode(q, kc, vc, L, out=out, workspace=ws))
        res[f"gqa_decode_B1_L{L}_16q4kv_D256"] = {"us": us, "GBps": round(gqa_bytes(1, Hq, Hkv, D, L) / us / 1e3, 1)}
        del kc, vc
    for S, Hq, Hkv, D in ((512, 32, 8, 128), (512, GQA_HQ, GQA_HKV, GQA_D)):   # prompt prefill
        qq = torch.randn((S, Hq * D), generator=g, **bf)
        kk = torch.randn((S, Hkv * D), generator=g, **bf)
        vv = torch.randn((S, Hkv * D), generator=g, **bf)
        o = torch.empty_like(qq)
        us = timed(lambda: aila_amd.gqa_prefill(qq, kk, vv, Hq, Hkv, out=o))
        res[f"gqa_prefill_S{S}_{Hq}q{Hkv}kv_D{D}"] = {"us": us,
                                                       "tflops": round(4 * D * Hq * S * (S + 1) / 2 / us / 1e6, 1)}
    Hk, Hv, d = DN_HK, DN_HV, DN_D
    st = torch.empty((1, Hv, d, d), dtype=torch.float32, device="cuda").normal_(0, 0.02, generator=g)
    q = torch.randn((1, Hk, d), generator=g, **bf)
    k = torch.randn((1, Hk, d), generator=g, **bf)
    v = torch.randn((1, Hv, d), generator=g, **bf)
    a = torch.randn((1, Hv), generator=g, **bf)
    b = torch.randn((1, Hv), generator=g, **bf)
    o = torch.empty((1, Hv, d), **bf)
    res["deltanet_decode_B1"] = {"us": timed(lambda: aila_amd.deltanet_decode(q, k, v, a, b, st, out=o))}
    ch = 2 * Hk * d + Hv * d
    cs = torch.empty((1, 3, ch), dtype=torch.float32, device="cuda").normal_(generator=g)
    w = torch.randn((ch, 4), generator=g, **bf)
    nw = torch.ones(d, dtype=torch.float32, device="cuda")
    arr = torch.zeros((Hk,), dtype=torch.int32, device="cuda")
    heads = torch.zeros((1,), dtype=torch.int32, device="cuda")
    x = dict(qkv=torch.randn((1, ch), generator=g, **bf), z=torch.randn((1, Hv * d), generator=g, **bf))
    lo = torch.empty((1, Hv * d), **bf)
    res["deltanet_layer_decode_B1"] = {"us": timed(lambda: aila_amd.deltanet_layer_decode(
        x["qkv"], x["z"], a, b, w, cs, 0, nw, st, Hk, out=lo, conv_heads=heads, arrivals=arr))}
    T = 512
    fused = torch.randn((1, T, ch + Hv * d + 2 * Hv), generator=g, **bf)
    lws = torch.empty(aila_amd.deltanet_layer_prefill_workspace_size(1, T, Hk, Hv), dtype=torch.uint8, device="cuda")
    lout = torch.empty((1, T, Hv * d), **bf)
    zc, ac = ch + Hv * d, ch + Hv * d + Hv
    res[f"deltanet_layer_prefill_T{T}"] = {"us": timed(lambda: aila_amd.deltanet_layer_prefill(
        fused[:, :, :ch], fused[:, :, ch:zc], fused[:, :, zc:ac], fused[:, :, ac:], w, cs, 0, nw, st, Hk, out=lout,
        workspace=lws))}
    return res


# ------------------------------------------------------------ CPU baseline --
def cpu_baseline(min_seconds=10.0):
    """The scalar oracle (fast-math build, OpenMP over heads) on the host
    cores: one 3:1 layer group of config 5 (3 DeltaNet layers + 1 GQA layer
    with the reference's split-K tile 128), batch 1, L = 32768, repeated
    until ~min_seconds of CPU work; GB/s of the same algorithmic bytes."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(0xA11A + 4)

    def bf16(shape):
        x = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
        return (x.view(np.uint32) >> 16).astype(np.uint16).reshape(shape)

    L = L5
    q = bf16((1, GQA_HQ, GQA_D))
    kc = bf16((1, GQA_HKV, L, GQA_D))
    vc = bf16((1, GQA_HKV, L, GQA_D))
    dn = [dict(q=bf16((1, 1, DN_HK, DN_D)), k=bf16((1, 1, DN_HK, DN_D)), v=bf16((1, 1, DN_HV, DN_D)),
               a=bf16((1, 1, DN_HV)), b=bf16((1, 1, DN_HV)),
               S=(rng.standard_normal((1, DN_HV, DN_D, DN_D), dtype=np.float32) * 0.02)) for _ in range(3)]
    lib = oracle.lib(fast=True)
    threads = oracle.num_threads(fast=True)

    def one():
        oracle.attention_decode_splitk(q, kc, vc, 1, GQA_HQ, GQA_HKV, GQA_D, L, L, 128, fast=True)
        for x in dn:
            oracle.deltanet_recurrent(x["q"], x["k"], x["v"], x["a"], x["b"], x["S"], 1, 1, DN_HK,
                                      DN_HV, DN_D, DN_D, fast=True)

    one()
    times = []
    t_end = time.perf_counter() + min_seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    byts = gqa_bytes(1, GQA_HQ, GQA_HKV, GQA_D, L) + 3 * deltanet_bytes(1, DN_HK, DN_HV, DN_D, DN_D)
    del lib
    return {"value": round(byts / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"oracle/liboracle_fast.so (-O3 -ffast-math, OpenMP {threads} threads): one config-5 "
                       f"layer group (1 GQA layer split-K tile 128 + 3 DeltaNet layers), batch 1, L={L}; "
                       f"median of {len(times)} runs ({sum(times):.1f} s)"),
            "seconds_per_group": round(t, 4),
            "config5_step_extrapolation": (
                f"the config-5 step is 8 such groups for each of 8 sequences: {64 * t:.2f} s per step at this "
                "rate (work and bytes both scale linearly with layers and batch, so the GB/s is the same)")}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_configs(runs=5):
    """The reference math (the scalar oracle, fast-math build, OpenMP) on the
    host cores for configs 2, 3 and 4, median of `runs` runs after one
    warm-up each. Baseline, not target. Config 2 runs the reference's naive
    3-pass prefill (AttentionOps.cpp:769-841) on the first 1024 tokens (a
    quarter of the causal FLOPs) and reports the FLOP rate; configs 3 and 4
    run the sequential recurrence (Qwen35HybridTextBackend.cpp:1729-1780)
    at full shape (config 3: all 2048 steps per run)."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(0xA11A)

    def bf16(shape):
        x = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
        return (x.view(np.uint32) >> 16).astype(np.uint16).reshape(shape)

    def med(fn):
        fn()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    threads = oracle.num_threads(fast=True)
    res = {"note": "baseline, not target", "cpu_model": cpu_model(), "threads": threads, "runs": runs,
           "build": "oracle/liboracle_fast.so (-O3 -ffast-math, OpenMP)"}
    # config 2: naive prefill on a 1024-token prefix (causal FLOPs scale as S^2)
    S, Hq, Hkv, D = 1024, 32, 8, 128
    q, k, v = bf16((S, Hq * D)), bf16((S, Hkv * D)), bf16((S, Hkv * D))
    t = med(lambda: oracle.attention_prefill_naive(q, k, v, S, Hq, Hkv, D, fast=True))
    fl = 4 * D * Hq * S * (S + 1) / 2
    full = 4 * D * Hq * 2048 * 2049 / 2
    res["config2_prefill"] = {"sample": "S=1024 prefix of config 2 (Hq=32 Hkv=8 D=128, causal, naive 3-pass)",
                              "seconds": round(t, 4), "gflops": round(fl / t / 1e9, 2),
                              "config2_seconds_at_that_rate": round(full / (fl / t), 3)}
    # config 3: the full 2048 sequential steps at B=32, H=16
    B, H, d, T = 32, 16, 128, 2048
    x = [bf16((B, T, H, d)) for _ in range(3)]
    a, b = bf16((B, T, H)), bf16((B, T, H))
    S0 = rng.standard_normal((B, H, d, d), dtype=np.float32) * 0.02
    t = med(lambda: oracle.deltanet_recurrent(x[0], x[1], x[2], a, b, S0, B, T, H, H, d, d, fast=True))
    res["config3_deltanet_decode"] = {"sample": "2048 sequential steps, B=32 H=16 dk=dv=128",
                                      "seconds": round(t, 3), "us_per_step": round(t / T * 1e6, 1)}
    del x, a, b
    # config 4: full sequence, sequential recurrence
    T, Hk, Hv = 4096, 16, 32
    x = [bf16((1, T, Hk, d)), bf16((1, T, Hk, d)), bf16((1, T, Hv, d))]
    a, b = bf16((1, T, Hv)), bf16((1, T, Hv))
    S0 = np.zeros((1, Hv, d, d), np.float32)
    t = med(lambda: oracle.deltanet_recurrent(x[0], x[1], x[2], a, b, S0, 1, T, Hk, Hv, d, d, fast=True))
    res["config4_deltanet_prefill"] = {"sample": "T=4096 Hk=16 Hv=32 dk=dv=128, sequential recurrence",
                                       "seconds": round(t, 4), "tok_per_s": round(T / t)}
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-sub", action="store_true", help="skip the config 1-4 sub-metrics")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile-kernel", nargs="?", const="gqa_decode", default=None,
                    choices=["gqa_decode", "gqa_prefill", "deltanet_decode", "deltanet_prefill", "paged_decode",
                             "deltanet_layer_decode", "deltanet_layer_prefill", "decode_prep", "fused_prep_decode",
                             "stack", "stack_full", "prefill_cached", "single_sequence"],
                    help="only run one kernel 20 times (default: the dominant config-5 GQA decode "
                         "layer, plus a 1 GiB device copy for counter calibration), for rocprofv3")
    ap.add_argument("--write-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/gqa_decode_config5_traffic.json from the two counter runs and exit")
    args = ap.parse_args()
    if args.write_traffic:
        write_traffic(*args.write_traffic)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path "
              "has no multi-GPU mode in this build.", file=sys.stderr)
        sys.exit(2)
    import torch

    import aila_amd
    aila_amd.lib()   # fail loudly if the HIP library is missing
    assert torch.cuda.is_available(), "bench.py needs a HIP device"

    if args.profile_kernel:
        r = {"gqa_decode": profile_kernel, "gqa_prefill": lambda t, a: sub_prefill(t, a, reps=20),
         "deltanet_decode": lambda t, a: sub_deltanet_decode(t, a, steps=320),
         "deltanet_prefill": lambda t, a: sub_deltanet_prefill(t, a, reps=20),
         "deltanet_layer_decode": lambda t, a: sub_deltanet_layer_decode(t, a, steps=320),
         "deltanet_layer_prefill": lambda t, a: sub_deltanet_layer_prefill(t, a, reps=10),
         "decode_prep": lambda t, a: sub_decode_prep(t, a, reps=20),
         "paged_decode": lambda t, a: sub_paged_decode(t, a),
         "fused_prep_decode": lambda t, a: sub_fused_prep_decode(t, a),
         "prefill_cached": lambda t, a: sub_prefill_cached(t, a),
         "single_sequence": lambda t, a: sub_single_sequence(t, a),
         "stack": lambda t, a: {k: v for k, v in bench_config5(t, a, 32, 4).items() if k != "W"},
         "stack_full": lambda t, a: bench_config5_full_layers(t, a, build_config5(t, a, 32, 4), 32, 4),
         }[args.profile_kernel](torch, aila_amd)
        if r:
            log(f"[profile] {args.profile_kernel}: {json.dumps(r)}")
        return
    log(f"[bench] config 5: {args.warmup} warmup + {args.steps} timed steps")
    device = device_info(torch)
    clocks = ClockSampler(torch)
    r5 = bench_config5(torch, aila_amd, args.steps, args.warmup, sampler=clocks)
    device["during_timed_steps"] = clocks.summary()
    log(f"[bench] device {device}")
    value = r5["step_bytes"] / (r5["ms"] * 1e-3) / 1e9
    log(f"[bench] config 5: {r5['ms']:.3f} ms/step, {value:.0f} GB/s")
    roof = roofline_gqa(torch, aila_amd, r5["W"])
    log(f"[bench] roofline gqa_decode: {roof['achieved']} GB/s ({roof['frac']*100:.1f}%)")
    full = bench_config5_full_layers(torch, aila_amd, r5["W"], args.steps, args.warmup)
    log(f"[bench] config 5 with whole layers: {full['ms_per_step']} ms/step, {full['GBps']} GB/s")
    del r5["W"]
    torch.cuda.empty_cache()
    sub = {"config5_full_layers": full}
    if not args.no_sub:
        sub["gqa_prefill"] = sub_prefill(torch, aila_amd)
        log(f"[bench] prefill {sub['gqa_prefill']}")
        sub["prefill_cached"] = sub_prefill_cached(torch, aila_amd)
        log(f"[bench] prefill cached {sub['prefill_cached']}")
        sub["deltanet_decode"] = sub_deltanet_decode(torch, aila_amd)
        log(f"[bench] deltanet decode {sub['deltanet_decode']}")
        sub["deltanet_layer_decode"] = sub_deltanet_layer_decode(torch, aila_amd)
        log(f"[bench] deltanet layer decode {sub['deltanet_layer_decode']}")
        sub["deltanet_prefill"] = sub_deltanet_prefill(torch, aila_amd)
        sub["deltanet_layer_prefill"] = sub_deltanet_layer_prefill(torch, aila_amd)
        log(f"[bench] deltanet layer prefill {sub['deltanet_layer_prefill']}")
        log(f"[bench] deltanet prefill {sub['deltanet_prefill']}")
        sub["gqa_decode_cfg1"] = sub_decode_cfg1(torch, aila_amd)
        sub["paged_decode"] = sub_paged_decode(torch, aila_amd)
        log(f"[bench] paged decode {sub['paged_decode']}")
        sub["decode_prep"] = sub_decode_prep(torch, aila_amd)
        log(f"[bench] decode prep {sub['decode_prep']}")
        sub["fused_prep_decode"] = sub_fused_prep_decode(torch, aila_amd)
        log(f"[bench] fused prep+decode {sub['fused_prep_decode']}")
        sub["single_sequence"] = sub_single_sequence(torch, aila_amd)
        log(f"[bench] single sequence {sub['single_sequence']}")
        log(f"[bench] decode cfg1 {sub['gqa_decode_cfg1']}")
    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline ...")
        cpu = cpu_baseline(args.cpu_seconds)
        cpu["cpu_model"] = cpu_model()
        log(f"[bench] CPU baseline {cpu['value']} GB/s on {cpu['cores']} threads")
        if not args.no_sub:
            sub["cpu_baseline_configs"] = cpu_baseline_configs()
            log(f"[bench] CPU baselines configs 2-4 {sub['cpu_baseline_configs']}")
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r5["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("config 5: Qwen3.5-4B-shaped hybrid attention stack decode, 24 Gated DeltaNet "
                         "(16qk/32v heads, dk=dv=128, fp32 state) + 8 GQA (16q/4kv, D=256, bf16 KV) layers"),
            "batch": B5, "context": r5["L_first"], "layers": N_LAYERS,
            "step_bytes": int(r5["step_bytes"]), "gqa_step_bytes": int(r5["gqa_step_bytes"]),
            "deltanet_step_bytes": int(r5["dn_step_bytes"]), "parallelism": "single GPU",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "device": device,
        "sub": sub,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
