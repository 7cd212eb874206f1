#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X (config 3 of the baseline: the HBM-roofline target).

Workload ("config3"): Llama-3-8B attention shape, 32 query / 8 KV heads, head dim 128, bf16,
batch 16, per-head spectral layout (8 groups, rank 128, row = b*8 + g), cache of 8192 tokens
growing by one token per step, retained dims r ~ clipped Beta with mean 0.29 and tokens 0-3
plus a seeded 5% forced to 128. Synthetic data generated on the device; the packed cache and all
per-step inputs are resident in HBM before the timed region.

One step = for each of 4 independent layer caches (a model's decode step runs all its layers),
the decode append of K and V for all 128 rows + the router decision + decode attention (long
route: the split-K kernel with two-stage semantics, which also merges the splits and projects
through the V basis). Four layers (~190 MB of packed cache each) keep a layer's cache from
staying in the 256 MB last-level cache between its calls, so the attention streams from HBM.

Output: one JSON line. ``value`` is decode-attention GB/s: algorithmic bytes of the attention
(packed K/V coefficients read once, int32 lengths, unique bases, q and output) divided by the
GPU time of the attention launches, summed over the timed steps (HIP events on the stream the
kernels run on, one pair around each step's back-to-back attention launches). ``roofline`` is
the split kernel (one launch per call); ``cpu_baseline`` times the masked-dimension CPU path on
a bounded sample of the same inputs. Beside them:
``cutoff_head`` (the cutoff head at the decode shape), ``prefill_attention`` (config 5's prompt
shape) and ``e2e`` (config 5: greedy generation with a random-init Llama-3-8B, compressed
against uncompressed cache).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Config3:
    name = "config3"
    B, G, Hq, Dh, R = 16, 8, 32, 128, 128
    S0 = 8192
    mean = 0.29
    theta = 500000.0
    dtype = torch.bfloat16
    force_first = 4
    force_frac = 0.05


class Config2:
    """Config 2 shape for one layer (the 32-layer stack repeats it): fp16, B=4, S=480."""
    name = "config2_layer"
    B, G, Hq, Dh, R = 4, 8, 32, 128, 128
    S0 = 480
    mean = 0.47
    theta = 500000.0
    dtype = torch.float16
    force_first = 0
    force_frac = 0.0


def build_workload(cfg, total_steps, dev, seed=1234):
    from dynakv_amd.kernels.compressed_cache import CustomDynamicCache
    from dynakv_amd.synthetic import device_lengths, random_orthogonal

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    rows = cfg.B * cfg.G
    S_all = cfg.S0 + total_steps
    lk = device_lengths(rows, S_all, cfg.R, cfg.mean, gen, dev, cfg.force_first, cfg.force_frac)
    lv = device_lengths(rows, S_all, cfg.R, cfg.mean, gen, dev, cfg.force_first, cfg.force_frac)
    rng = np.random.default_rng(seed)
    kb = np.stack([random_orthogonal(cfg.R, rng).T for _ in range(cfg.G)])
    vb = np.stack([random_orthogonal(cfg.R, rng).T for _ in range(cfg.G)])
    k_basis = torch.from_numpy(kb).to(dev, cfg.dtype).contiguous()
    v_basis = torch.from_numpy(vb).to(dev, cfg.dtype).contiguous()
    cache = CustomDynamicCache()
    kx = torch.randn((rows, cfg.S0, cfg.R), generator=gen, device=dev).to(cfg.dtype)
    vx = torch.randn((rows, cfg.S0, cfg.R), generator=gen, device=dev).to(cfg.dtype)
    cache.update_sp(kx, lk[:, : cfg.S0].contiguous(), vx, lv[:, : cfg.S0].contiguous(), cfg.R, 0,
                    cfg.R)
    del kx, vx
    steps_k = torch.randn((total_steps, rows, 1, cfg.R), generator=gen, device=dev).to(cfg.dtype)
    steps_v = torch.randn((total_steps, rows, 1, cfg.R), generator=gen, device=dev).to(cfg.dtype)
    q = torch.randn((total_steps, cfg.B, cfg.Hq, cfg.Dh), generator=gen, device=dev).to(cfg.dtype)
    lk_steps = lk[:, cfg.S0:].t().contiguous().unsqueeze(-1)  # (steps, rows, 1)
    lv_steps = lv[:, cfg.S0:].t().contiguous().unsqueeze(-1)
    # host copies of the per-token counts for byte accounting (outside any timed region)
    lk_h = lk.to(torch.int64).cpu().numpy()
    lv_h = lv.to(torch.int64).cpu().numpy()
    torch.cuda.synchronize(dev)
    return dict(cache=cache, k_basis=k_basis, v_basis=v_basis, steps_k=steps_k, steps_v=steps_v,
                q=q, lk_steps=lk_steps, lv_steps=lv_steps, lk_h=lk_h, lv_h=lv_h, gen=gen)


def attention_bytes(cfg, lk_h, lv_h, S, split_only=False):
    """Algorithmic HBM bytes of one decode-attention call at cache length S: packed K and V
    coefficients read once, one int32 length per token, row and K|V, the unique bases, q and the
    output. ``split_only``: what the split kernel alone must move (no V basis, no output)."""
    elt = 2
    coef = elt * (int(lk_h[:, :S].sum()) + int(lv_h[:, :S].sum()))
    lens = 8 * cfg.B * cfg.G * S
    basis = cfg.G * cfg.R * cfg.Dh * elt
    q = cfg.B * cfg.Hq * cfg.Dh * elt
    if split_only:
        return coef + lens + basis + q
    return coef + lens + 2 * basis + 2 * q


class SplitKRunner:
    """Launches dkv_decode_splitk on the current stream (the split kernel merges its own splits;
    the library times it with HIP events on that stream). The RoPE table and the workspace are
    built once, before any timed step."""

    def __init__(self, cfg, dev, max_S):
        from dynakv_amd import _lib
        from dynakv_amd.kernels.decode import rope_table, workspace

        self.lib = _lib.load()
        self._lib = _lib
        self.cfg = cfg
        self.dev = dev
        st = torch.cuda.current_stream(dev).cuda_stream
        # the automatic split length changes with S (fewer, longer splits as the cache grows),
        # so the workspace is sized for the largest need over the lengths the run visits
        nfl = max(self.lib.dkv_splitk_workspace_floats(cfg.B, cfg.Hq, cfg.G, S, cfg.R, 0)
                  for S in range(cfg.S0, max_S + 1))
        self.ws = workspace(dev, st, int(nfl))
        self.rope, self.rope_tiles = rope_table(dev, st, cfg.theta, max_S)
        self.out = torch.empty((cfg.B, cfg.Hq, cfg.Dh), dtype=cfg.dtype, device=dev)

    def run(self, q, fk, fv, lk, ok, lv, ov, kb, vb, route):
        cfg, L = self.cfg, self._lib
        S = lk.shape[1]
        st = torch.cuda.current_stream(self.dev)
        args = (st.cuda_stream, route, L.dtype_code(cfg.dtype),
                q.data_ptr(), q.stride(0), q.stride(1),
                kb.data_ptr(), kb.stride(0), kb.stride(1), vb.data_ptr(), vb.stride(0), vb.stride(1),
                fk.data_ptr(), fk.stride(0), fv.data_ptr(), fv.stride(0),
                lk.data_ptr(), ok.data_ptr(), lk.stride(0), lk.stride(1),
                lv.data_ptr(), ov.data_ptr(), lv.stride(0), lv.stride(1),
                self.rope.data_ptr(), self.rope_tiles, self.ws.data_ptr(), self.ws.numel(),
                self.out.data_ptr(), self.out.stride(0), self.out.stride(1),
                L.dtype_code(cfg.dtype), cfg.B, cfg.Hq, cfg.G, cfg.G, S, cfg.R, cfg.Dh, 0)
        L.check(self.lib.dkv_decode_splitk(*args), "dkv_decode_splitk")
        return self.out


def run_gpu(cfg, steps, warmup, dev, layers, lib_profile=False, prewarm_s=0.0):
    """Time ``steps`` decode steps; each step appends K and V to every one of ``layers``
    independent layer caches (a model's decode step runs all its layers) and then runs their
    decode attention back to back (router + attention launch per layer). Several layers keep a
    layer's cache from staying resident in the 256 MB last-level cache between its calls, so
    the attention streams its coefficients from HBM.

    Attention GPU time: one pair of HIP events (torch events on the stream the kernels are
    launched on) around each step's ``layers`` attention launches, so the figure is kernel time
    plus the gaps between back-to-back launches, without an event pair's own cost per launch.
    When a launch takes less GPU time than the host needs to submit the next one (short
    caches), those gaps are host time. ``lib_profile`` also records the library's own event
    pair around every launch (``dkv_profile_begin`` / ``dkv_profile_end``, one session per
    route): ``lib_ms`` maps each route to (GPU ms summed over its launches, launches).

    ``prewarm_s``: after the first warmup step, its attention launches are repeated (untimed, on
    the caches as that step left them, no appends) for that many seconds of wall time, so that
    the timed steps run at the GPU's sustained clocks: from idle the same launches take ~20%
    longer over the first ~100 ms of load."""
    from dynakv_amd import _lib
    from dynakv_amd.kernels.router import KernelPolicy

    total = steps + warmup
    _log(f"building {cfg.name} workload (B={cfg.B}, S0={cfg.S0}, steps={total}, layers={layers})")
    Ws = [build_workload(cfg, total, dev, seed=1234 + 7919 * l) for l in range(layers)]
    runner = SplitKRunner(cfg, dev, cfg.S0 + total + 16)
    policy = KernelPolicy()
    R = cfg.R

    def append(W, i):
        cache = W["cache"]
        tabs = cache.update_sp(W["steps_k"][i], W["lk_steps"][i], W["steps_v"][i],
                               W["lv_steps"][i], R, 0, R)
        return tabs, cache.get_seq_length_sp(0)

    def attend(W, i, tabs, L):
        fk, fv, lk, lv, ok, ov = tabs
        route = (_lib.DKV_ROUTE_FUSED if policy.select(L) == "short_fused"
                 else _lib.DKV_ROUTE_TWO_STAGE)
        runner.run(W["q"][i], fk, fv, lk, ok, lv, ov, W["k_basis"], W["v_basis"], route)

    last = {}

    def step(i, events=None):
        apps = [append(W, i) for W in Ws]
        last["tabs"], last["len"], last["i"], last["apps"] = apps[0][0], apps[0][1], i, apps
        if events is not None:
            events[0].record()
        for W, (tabs, L) in zip(Ws, apps):
            attend(W, i, tabs, L)
        if events is not None:
            events[1].record()
        return [L for _, L in apps]

    lib = _lib.load()
    lib_ms = {}
    cur = [None]  # route of the open library-profiling session

    def lib_session(route):
        if cur[0] == route:
            return
        if cur[0] is not None:
            split_ms, merge_ms, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int()
            _lib.check(lib.dkv_profile_end(ctypes.byref(split_ms), ctypes.byref(merge_ms),
                                           ctypes.byref(n)), "dkv_profile_end")
            t, c = lib_ms.get(cur[0], (0.0, 0))
            lib_ms[cur[0]] = (t + split_ms.value + merge_ms.value, c + n.value)
        cur[0] = route
        if route is not None:
            _lib.check(lib.dkv_profile_begin(steps * layers), "dkv_profile_begin")

    prewarm_calls = 0
    for i in range(warmup):
        step(i)
        if i == 0 and prewarm_s > 0:
            torch.cuda.synchronize(dev)
            t_end = time.perf_counter() + prewarm_s
            while time.perf_counter() < t_end:
                for W, (tabs, L) in zip(Ws, last["apps"]):
                    attend(W, i, tabs, L)
                prewarm_calls += layers
                if prewarm_calls % (8 * layers) == 0:  # keep the host a few launches ahead
                    torch.cuda.synchronize(dev)
    torch.cuda.synchronize(dev)
    _log("timed region")
    lens, evs = [], []
    t0 = time.perf_counter()
    for j in range(steps):
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        if lib_profile:  # the route of this step's launches, from the length after its append
            lib_session(policy.select(Ws[0]["cache"].get_seq_length_sp(0) + 1))
        lens.extend(enumerate(step(warmup + j, ev)))
        evs.append(ev)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    if lib_profile:
        lib_session(None)
    attn_ms = sum(e0.elapsed_time(e1) for e0, e1 in evs)
    step_bytes = [attention_bytes(cfg, Ws[l]["lk_h"], Ws[l]["lv_h"], L) for l, L in lens]
    tot_bytes = float(sum(step_bytes))
    calls = steps * layers
    # fused merge (one launch per call) unless the call has more units than arrival counters
    units = cfg.B * cfg.G
    step_ms = [e0.elapsed_time(e1) for e0, e1 in evs]
    step_len = [lens[j * layers][1] for j in range(steps)]  # layer 0's length at each step
    return dict(
        wall_s=wall, attn_ms=attn_ms, split_ms=attn_ms, merge_ms=0.0, calls=calls,
        prewarm_calls=prewarm_calls,
        step_ms=step_ms, step_len=step_len, lib_ms=lib_ms,
        runner=runner, last_tabs=last["tabs"], last_len=last["len"],
        last_q=Ws[0]["q"][last["i"]],
        merged_in_split=units <= 16384,
        bytes_total=tot_bytes, bytes_per_call=tot_bytes / calls,
        split_bytes_per_call=float(sum(attention_bytes(cfg, Ws[l]["lk_h"], Ws[l]["lv_h"], L,
                                                       split_only=True) for l, L in lens)) / calls,
        final_len=Ws[0]["cache"].get_seq_length_sp(0),
        syncs=sum(W["cache"].device_syncs for W in Ws),
        cache=Ws[0]["cache"], workload=Ws[0],
    )


def bench_dense_same_shape(dev, S=8192, B=16, Hkv=8, hpg=4, layers=4, steps=20, prewarm_s=0.0):
    """The uncompressed baseline's decode attention (``dkv_decode_dense``) at the main workload's
    shape: every token's rotated key and value at 128 dims (the reference's original model,
    ``scripts/benchmark_throughput.py``), ``layers`` caches cycled so that none stays in the
    last-level cache, their launches timed back to back with one event pair per step as the
    compressed workload is (after the same untimed ``prewarm_s`` of repeated launches). Bytes:
    K and V of every token, q and the output."""
    from dynakv_amd.kernels.decode import dense_decode_attention

    g = torch.Generator(device=dev)
    g.manual_seed(99)
    rows = B * Hkv
    caches = [(torch.randn((rows, S * 128), generator=g, device=dev).to(torch.bfloat16),
               torch.randn((rows, S * 128), generator=g, device=dev).to(torch.bfloat16))
              for _ in range(layers)]
    q = torch.randn((B, Hkv * hpg, 128), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    for _ in range(2):
        for k, v in caches:
            dense_decode_attention(q, k, v, S, out=out)
    torch.cuda.synchronize(dev)
    t_end, n = time.perf_counter() + prewarm_s, 0
    while time.perf_counter() < t_end:
        for k, v in caches:
            dense_decode_attention(q, k, v, S, out=out)
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize(dev)
    torch.cuda.synchronize(dev)
    evs = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for k, v in caches:
            dense_decode_attention(q, k, v, S, out=out)
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize(dev)
    us = sum(a.elapsed_time(b) for a, b in evs) * 1e3 / (steps * layers)
    nbytes = 2 * rows * S * 128 * 2 + 2 * q.numel() * 2
    del caches
    torch.cuda.empty_cache()
    return {"kernel": "dense_decode_kernel<bf16>", "batch": B, "kv_heads": Hkv,
            "q_heads": Hkv * hpg, "cache_len": S, "bytes_per_call": nbytes,
            "us_per_call": round(us, 3), "achieved_gbs": round(nbytes / (us * 1e-6) / 1e9, 2),
            "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def graph_us_per_call(fn, dev, n=20, reps=5):
    """GPU time per call of ``fn`` replayed ``n`` times back to back from a HIP graph (no host
    work between the launches), the best of ``reps`` replays. ``fn`` launches on torch's
    current stream; it is warmed up on the capture stream first (its workspaces are per
    stream)."""
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(n):
            fn()
    torch.cuda.synchronize(dev)
    best = float("inf")
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            e0.record()
            g.replay()
            e1.record()
        torch.cuda.synchronize(dev)
        best = min(best, e0.elapsed_time(e1) * 1e3 / n)
    del g
    return best


def bench_config2(dev, steps=100, warmup=10, layers=4, prewarm_s=0.0):
    """Config 2 as one layer of its 32-layer stack (fp16, B=4, 8 KV groups x rank 128, mean
    retention 0.47): ``steps`` decode steps from 480 tokens on, so the router's switch at 500
    tokens is crossed (fused route below it, two-stage from it on), each step appending to
    ``layers`` independent layer caches and timing their back-to-back attention launches as the
    main workload does. Reports us per layer-step overall and per route, and the algorithmic
    bytes per launch against HBM peak (a latency-bound launch: 4.4-5.4 MB per call).

    A launch here takes less GPU time than the host needs to submit it from Python, so the
    step's event pair measures the host's pace; the figures are the library's event pairs
    around each launch (GPU time per launch), with the host-paced figures beside them."""
    cfg = Config2
    r = run_gpu(cfg, steps, warmup, dev, layers, lib_profile=True, prewarm_s=prewarm_s)
    calls = r["calls"]
    lib_ms = r["lib_ms"]
    lib_total = sum(t for t, _ in lib_ms.values())
    lib_calls = sum(c for _, c in lib_ms.values())
    us = lib_total * 1e3 / lib_calls
    per_route = {k: round(t * 1e3 / c, 3) for k, (t, c) in lib_ms.items() if c}
    fused = [ms for ms, L in zip(r["step_ms"], r["step_len"]) if L < 500]
    two = [ms for ms, L in zip(r["step_ms"], r["step_len"]) if L >= 500]
    per = lambda v: round(sum(v) * 1e3 / (len(v) * layers), 3) if v else None  # noqa: E731
    bpc = r["bytes_per_call"]
    return {
        "workload": cfg.name, "batch": cfg.B, "q_heads": cfg.Hq, "kv_heads": cfg.G,
        "rank": cfg.R, "dtype": "fp16", "mean_retention": cfg.mean,
        "cache_len_start": cfg.S0, "cache_len_end": r["final_len"], "steps": steps,
        "layers_per_step": layers,
        "us_per_layer_step": round(us, 3),
        "us_per_layer_step_fused_route": per_route.get("short_fused"),
        "us_per_layer_step_two_stage_route": per_route.get("long_two_stage"),
        "bytes_per_launch": round(bpc),
        "achieved_gbs": round(bpc / (us * 1e-6) / 1e9, 2),
        "frac_hbm_peak": round(bpc / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "timing": "the library's HIP event pair around each attention launch (dkv_profile_begin"
                  " / dkv_profile_end): GPU time per launch",
        "graph_replayed": _config2_graph(dev, cfg, r),
        "host_paced_us_per_layer_step": round(r["attn_ms"] * 1e3 / calls, 3),
        "host_paced_us_per_layer_step_fused_route": per(fused),
        "host_paced_us_per_layer_step_two_stage_route": per(two),
        "host_paced_timing": "HIP events around each step's back-to-back attention launches "
                             "(as the main workload); here the host's submission rate",
    }


def _config2_graph(dev, cfg, r):
    """Config 2 at its final length, 20 launches replayed from a HIP graph: the split kernel
    on the last step's cache (its route at that length) and the uncompressed baseline's decode
    kernel (dkv_decode_dense) on a dense cache of the same shape: the floor of a split-and-merge
    decode launch with no reconstruction."""
    from dynakv_amd import _lib
    from dynakv_amd.kernels.decode import dense_decode_attention

    fk, fv, lk, lv, ok, ov = r["last_tabs"]
    W = r["workload"]
    q = r["last_q"]
    S = int(r["last_len"])
    route = _lib.DKV_ROUTE_FUSED if S < 500 else _lib.DKV_ROUTE_TWO_STAGE
    runner = r["runner"]
    comp = graph_us_per_call(
        lambda: runner.run(q, fk, fv, lk, ok, lv, ov, W["k_basis"], W["v_basis"], route), dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    kd = torch.randn((cfg.B * cfg.G, (S + 16) * cfg.Dh), generator=gen, device=dev).to(cfg.dtype)
    vd = torch.randn((cfg.B * cfg.G, (S + 16) * cfg.Dh), generator=gen, device=dev).to(cfg.dtype)
    out = torch.empty((cfg.B, cfg.Hq, cfg.Dh), dtype=cfg.dtype, device=dev)
    dense = graph_us_per_call(lambda: dense_decode_attention(q, kd, vd, S, out=out), dev)
    return {"cache_len": S, "compressed_us_per_launch": round(comp, 3),
            "dense_us_per_launch": round(dense, 3),
            "timing": "20 launches replayed from a HIP graph, best of 5 replays"}


def cpu_baseline(cfg, W, cache, budget_s: float):
    """Masked-dimension CPU path (oracle.masked_dim, fp32 torch) on batch row 0 of the same
    cache: dense masked coefficients for the 8 groups, block-diagonal joint basis, full
    reconstruction + RoPE + eager attention per step."""
    from oracle import masked_dim as M

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    G, R, Dh = cfg.G, cfg.R, cfg.Dh
    dk, dv = cache.get_origin_states(R, 0)  # (rows, S, R) on the device
    S = dk.shape[1]
    ck = dk[:G].float().cpu().permute(1, 0, 2).reshape(1, S, G * R).contiguous()
    cv = dv[:G].float().cpu().permute(1, 0, 2).reshape(1, S, G * R).contiguous()
    Uk = M.block_diag_up(W["k_basis"].float().cpu())
    Uv = M.block_diag_up(W["v_basis"].float().cpu())
    q = W["q"][0][:1].float().cpu()
    n, t0 = 0, time.perf_counter()
    while True:
        M.decode_attention(q, ck, cv, Uk, Uv, G, cfg.theta)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 50:
            break
    per_call = el / n
    lk_h, lv_h = W["lk_h"][:G], W["lv_h"][:G]
    bytes_row = 2 * (int(lk_h[:, :S].sum()) + int(lv_h[:, :S].sum())) + 8 * G * S \
        + 2 * G * R * Dh * 2 + 2 * cfg.Hq * Dh * 2
    try:
        model = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        model = next((l.split(":", 1)[1].strip() for l in model.splitlines()
                      if l.startswith("Model name")), platform.processor())
    except Exception:
        model = platform.processor()
    return {
        "value": bytes_row / per_call / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"batch row 0 of 16 (8 KV groups, S={S}), {n} decode-attention calls of the "
                   f"masked-dimension fp32 torch path (dense 1024-d masked coefficients, "
                   f"block-diagonal basis), {per_call * 1e3:.1f} ms/call on {model}"),
        "ms_per_layer_step_full_batch_extrapolated": per_call * 1e3 * cfg.B,
    }


def bench_cutoff(cfg, dev, iters=50):
    """Cutoff head (reference kv_process_fused, compressed_attention.py:84-119) for K and V at
    this workload's decode shape: per-head (G groups of D = R dims) and the reference's joint
    head (one 1024-d group). Time per call from HIP events on the current stream, eager (host
    launch cost included) and replayed from a HIP graph (GPU time, as the reference's decode
    step replays the call), against the reference formula evaluated by torch's own GPU kernels
    (addmm, softmax, cumsum, flip, compare, sum, multiply) on the same inputs."""
    from dynakv_amd.kernels.cutoff import CutoffHead

    res = {}
    g = torch.Generator(device="cpu").manual_seed(99)
    for mode, G, D in (("per_head", cfg.G, cfg.R), ("joint", 1, cfg.G * cfg.Dh)):
        M = cfg.B
        W = [(torch.randn(G, D, D, generator=g) * 3 / D ** 0.5).to(dev, cfg.dtype) for _ in range(2)]
        b = [torch.randn(G, D, generator=g).to(dev, cfg.dtype) for _ in range(2)]
        head = CutoffHead(W[0] if G > 1 else W[0][0], b[0], W[1] if G > 1 else W[1][0], b[1],
                          groups=G)
        x = [torch.randn(M, 1, G * D, generator=g).to(dev, cfg.dtype) for _ in range(2)]

        def torch_ref():
            outs = []
            for t in range(2):
                xf = x[t].view(M, G, D).transpose(0, 1).contiguous()  # (G, M, D)
                lg = torch.baddbmm(b[t].unsqueeze(1), xf, W[t])
                mask = torch.softmax(lg, dim=-1).cumsum(dim=-1).flip(dims=[-1]) >= 0.1
                outs.append((xf * mask, mask.sum(dim=-1, dtype=torch.int32)))
            return outs

        for fn in (lambda: head.kv_process_fused(x[0], x[1]), torch_ref):
            for _ in range(5):
                fn()
        torch.cuda.synchronize(dev)
        times = {}
        for name, fn in (("dynakv", lambda: head.kv_process_fused(x[0], x[1])), ("torch", torch_ref)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                fn()
            e1.record()
            torch.cuda.synchronize(dev)
            times[name] = e0.elapsed_time(e1) * 1e3 / iters
        # The reference replays kv_process_fused under a CUDA graph (compressed_attention.py:
        # 321-334): the call captured 20 times in one HIP graph, replayed, gives its GPU time
        # without the host's per-call cost; one replay is checked against the eager result.
        per_graph = 20
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(3):
                head.kv_process_fused(x[0], x[1])
        torch.cuda.current_stream(dev).wait_stream(side)
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            gouts = [head.kv_process_fused(x[0], x[1]) for _ in range(per_graph)]
        gph.replay()
        torch.cuda.synchronize(dev)
        want = head.kv_process_fused(x[0], x[1])
        torch.cuda.synchronize(dev)
        graph_ok = all(torch.equal(a, b) for a, b in zip(gouts[-1][:4], want[:4]))
        reps = max(1, iters // per_graph)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            gph.replay()
        e1.record()
        torch.cuda.synchronize(dev)
        graph_us = e0.elapsed_time(e1) * 1e3 / (reps * per_graph)
        del gph, gouts
        nbytes = 2 * (G * D * D * 2 + G * D * 2 + 2 * M * G * D * 2 + M * G * 4)
        res[mode] = {
            "shape": f"M={M} tokens, G={G} x D={D}, K and V",
            "us_per_call": round(times["dynakv"], 2),
            "graph_us_per_call": round(graph_us, 2),
            "graph_replay_matches_eager": graph_ok,
            "torch_eager_us_per_call": round(times["torch"], 2),
            "algorithmic_bytes": nbytes,
            "gbs": round(nbytes / (graph_us * 1e-6) / 1e9, 1),
        }
    return res


def bench_prefill(dev, iters=10, B=4, S=2048, Hq=32, Hkv=8, dtype=torch.bfloat16):
    """Causal prefill attention at the config-5 prompt shape (B=4 prompts of 2048 tokens,
    Llama-3-8B heads): dkv_prefill_attention against torch's scaled_dot_product_attention on
    the same inputs (K/V repeated over the query heads for it). GPU time from events around
    ``iters`` back-to-back calls."""
    from dynakv_amd.kernels.prefill import prefill_attention

    g = torch.Generator(device="cpu").manual_seed(7)
    q = torch.randn(B, Hq, S, 128, generator=g).to(dev, dtype)
    k = torch.randn(B, Hkv, S, 128, generator=g).to(dev, dtype)
    v = torch.randn(B, Hkv, S, 128, generator=g).to(dev, dtype)
    kr = k.repeat_interleave(Hq // Hkv, dim=1).contiguous()
    vr = v.repeat_interleave(Hq // Hkv, dim=1).contiguous()
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def sdpa():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return torch.nn.functional.scaled_dot_product_attention(q, kr, vr, is_causal=True)

    fns = {"dynakv": lambda: prefill_attention(q, k, v, causal=True), "torch_sdpa": sdpa}
    times = {}
    for name, fn in fns.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        times[name] = e0.elapsed_time(e1) / iters
    flops = 2.0 * 2 * B * Hq * (S * (S + 1) / 2) * 128  # QK and PV over the causal triangle
    # agreement with torch on the same inputs (both in the compute dtype; torch's output is
    # itself rounded, so this is a cross-check, the oracle tests are the parity bar)
    ours = prefill_attention(q, k, v, causal=True, out_dtype=torch.float32)
    theirs = sdpa().float()
    diff = (ours - theirs).abs().max().item()
    return {
        "shape": f"B={B}, S={S}, {Hq}/{Hkv} heads, Dh 128, causal, {str(dtype).split('.')[-1]}",
        "max_abs_vs_torch_sdpa": float(f"{diff:.3e}"),
        "ms_per_call": round(times["dynakv"], 4),
        "tflops": round(flops / (times["dynakv"] * 1e-3) / 1e12, 1),
        "torch_sdpa_ms_per_call": round(times["torch_sdpa"], 4),
        "torch_sdpa_tflops": round(flops / (times["torch_sdpa"] * 1e-3) / 1e12, 1),
    }


def bench_joint(dev, iters=5, B=16, S=8192, R=1024, Hq=32, Hkv=8, mean=0.29,
                dtype=torch.bfloat16):
    """The reference's joint layout at the config-3 shape: one packed row per batch element with
    ranks up to 1024 shared by the 8 KV heads, k_up / v_up repeated to the 32 query heads as the
    reference ships them (compressed_attention.py:278-286), the router's long route
    (abx_sparse + avx semantics) through the MFMA kernels of ``kernels/joint.py``. GPU time from
    events around ``iters`` back-to-back calls; the scores kernel's MFMA work counted as
    launched (2 * 128 * 32 flop per rank chunk, token slot and KV head, each workgroup's tokens
    sorted by chunk count and every 16 sorted tokens run up to their longest token's chunks).
    The vector kernels (dkv_scores / dkv_av, what a joint layout ran on before) are timed on a
    2 x 512-token slice of the same data."""
    import math as _m

    from dynakv_amd import _lib
    from dynakv_amd.kernels import joint as J
    from dynakv_amd.synthetic import device_lengths

    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    lk = device_lengths(B, S, R, mean, gen, dev, 4, 0.05)
    lv = device_lengths(B, S, R, mean, gen, dev, 4, 0.05)

    def packed(lens):
        offs = torch.zeros_like(lens)
        offs[:, 1:] = torch.cumsum(lens, dim=1)[:, :-1]
        cap = int(lens.sum(dim=1).max().item())
        flat = torch.randn((B, cap), generator=gen, device=dev, dtype=torch.float32).to(dtype)
        return flat, offs.to(torch.int32).contiguous()

    fk, ok = packed(lk)
    fv, ov = packed(lv)
    kb = (torch.randn((Hkv, R, 128), generator=gen, device=dev) / _m.sqrt(R)).to(dtype)
    vb = (torch.randn((Hkv, R, 128), generator=gen, device=dev) / _m.sqrt(R)).to(dtype)
    k_up = kb.repeat_interleave(Hq // Hkv, dim=0).contiguous()
    v_up = vb.repeat_interleave(Hq // Hkv, dim=0).contiguous()
    q = torch.randn((B, Hq, 128), generator=gen, device=dev).to(dtype)
    theta = 500000.0

    def timed(fn, n):
        for _ in range(2):
            fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / n * 1e3  # us

    route = _lib.DKV_ROUTE_TWO_STAGE
    full = timed(lambda: J.joint_attention(q, fk, k_up, fv, v_up, lk, ok, lv, ov, theta=theta,
                                           route=route), iters)
    sc = J.joint_scores(q, k_up, fk, lk, ok, theta=theta, mode=0, out_dtype=dtype)
    t_sc = timed(lambda: J.joint_scores(q, k_up, fk, lk, ok, theta=theta, mode=0,
                                        out_dtype=dtype), iters)
    t_av = timed(lambda: J.joint_av(sc, v_up, fv, lv, ov, mode=0, out_dtype=dtype), iters)
    flops = J.joint_flops(lk, R, Hkv, B)
    dense_flops = 2.0 * B * S * Hkv * 128 * R
    useful_flops = 2.0 * 128 * Hkv * float(lk.clamp(0, R).sum().item())
    coef_bytes = 2 * int(lk.clamp(0, R).sum().item() + lv.clamp(0, R).sum().item())

    # the vector kernels on a slice: 2 rows x 512 tokens
    b2, s2 = 2, 512
    lib = _lib.load()
    lk2, ok2, lv2, ov2 = (t[:b2, :s2].contiguous() for t in (lk, ok, lv, ov))
    q2 = q[:b2].contiguous()
    st = _lib.stream_of(q2)
    sc2 = torch.empty((b2, Hq, s2), dtype=dtype, device=dev)
    out2 = torch.empty((b2, Hq, 128), dtype=dtype, device=dev)

    def vector_pass():
        lib.dkv_scores(st, 0, _lib.dtype_code(dtype), _lib.dtype_code(dtype), _lib.dtype_code(dtype),
                       q2.data_ptr(), q2.stride(0), q2.stride(1), k_up.data_ptr(), k_up.stride(0),
                       k_up.stride(1), Hq, fk.data_ptr(), fk.stride(0), lk2.data_ptr(),
                       lk2.stride(0), lk2.stride(1), ok2.data_ptr(), ok2.stride(0), ok2.stride(1),
                       sc2.data_ptr(), sc2.stride(0), sc2.stride(1), sc2.stride(2),
                       b2, Hq, s2, R, 128, _m.log(theta))
        lib.dkv_av(st, 0, _lib.dtype_code(dtype), _lib.dtype_code(dtype), _lib.dtype_code(dtype),
                   sc2.data_ptr(), sc2.stride(0), sc2.stride(1), sc2.stride(2), v_up.data_ptr(),
                   v_up.stride(0), v_up.stride(1), Hq, fv.data_ptr(), fv.stride(0),
                   lv2.data_ptr(), lv2.stride(0), lv2.stride(1), ov2.data_ptr(), ov2.stride(0),
                   ov2.stride(1), out2.data_ptr(), out2.stride(0), out2.stride(1),
                   b2, Hq, s2, R, 128)

    t_vec = timed(vector_pass, 2)
    t_mfma_slice = timed(lambda: J.joint_attention(q2, fk, k_up, fv, v_up, lk2, ok2, lv2, ov2,
                                                   theta=theta, route=route), 5)
    return {
        "shape": (f"B={B}, S={S}, joint rank {R} shared by {Hkv} KV heads, k_up/v_up repeated "
                  f"to {Hq} query heads, mean retention {mean}, {str(dtype).split('.')[-1]}, "
                  "long route"),
        "us_per_call": round(full, 1),
        "scores_us": round(t_sc, 1),
        "av_us": round(t_av, 1),
        "scores_mfma_tflops": round(flops / (t_sc * 1e-6) / 1e12, 1),
        "scores_mfma_peak_frac": round(flops / (t_sc * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "scores_flop_as_launched": flops,
        "reconstruction_flop_dense": dense_flops,
        "reconstruction_flop_useful": useful_flops,
        "scores_useful_peak_frac": round(useful_flops / (t_sc * 1e-6) / 1e12
                                         / MFMA_BF16_PEAK_TFLOPS, 4),
        "coefficient_bytes": coef_bytes,
        "vector_kernels_slice": {"slice": f"B={b2}, S={s2}", "us_per_call": round(t_vec, 1),
                                 "mfma_us_per_call": round(t_mfma_slice, 1)},
    }


def bench_e2e(dev, batches=(1, 2, 4), prompt_len=2048, new_tokens=100, models="all"):
    """Config 5: greedy generation with a random-init Llama-3-8B (bf16 N(0, 0.02) weights,
    per-head random orthogonal bases, cutoff heads set for mean retention 0.47) over the
    compressed cache, against the same weights with an uncompressed cache (the reference's
    original model: rotated keys and values at 128 dims, decode attention by the dense GQA
    kernel ``dkv_decode_dense``, the cache write and q rotation in one launch; prefill attention
    by torch's fused attention). tokens/s = batch * new tokens / wall time
    with prefill, as the reference's benchmark_throughput.py:73 counts it; decode-only tokens/s
    beside it. A third run keeps the dense cache but decodes through torch's fused
    ``scaled_dot_product_attention``, the attention of the reference's transformers baseline.
    All run eagerly (one launch per op, no graph capture). ``models``: "all", or a comma list
    of "compressed", "dense" and "sdpa" (one model alone, for a kernel trace of it)."""
    from dynakv_amd.model import CompressedLlama, DenseLlama, LlamaShape, RandomLlama

    want = {"compressed", "dense", "sdpa"} if models == "all" else set(models.split(","))
    shape = LlamaShape()
    model = RandomLlama(shape, device=dev, seed=5)
    comp = CompressedLlama(model) if "compressed" in want else None
    dense = (DenseLlama(model, max_len=prompt_len + new_tokens + 8)
             if "dense" in want else None)
    sdpa = (DenseLlama(model, max_len=prompt_len + new_tokens + 8, attention="sdpa")
            if "sdpa" in want else None)
    g = torch.Generator(device="cpu").manual_seed(11)
    res = {"model": "random-init Llama-3-8B shape (32 layers, 4096 hidden, 32/8 heads, FFN "
                    "14336, vocab 128256), bf16", "prompt_len": prompt_len,
           "new_tokens": new_tokens, "runs": []}
    # one short warm-up of each path (kernel loading, library handles)
    warm = torch.randint(0, shape.vocab, (1, 64), generator=g).to(dev)
    for m in (comp, dense, sdpa):
        if m is not None:
            m.generate(warm, 4)
    # a model left out of this run reports null
    empty = {"tokens_per_s": None, "decode_tokens_per_s": None, "prefill_s": None,
             "kv_bytes": None, "tokens": None}

    def rnd(v, n):
        return None if v is None else round(v, n)
    for B in batches:
        prompt = torch.randint(0, shape.vocab, (B, prompt_len), generator=g).to(dev)
        rc = comp.generate(prompt, new_tokens) if comp is not None else empty
        rd = dense.generate(prompt, new_tokens) if dense is not None else empty
        rs = sdpa.generate(prompt, new_tokens) if sdpa is not None else empty
        lens = ([int(c[1][:, :c[4]].float().mean().item()) for c in comp.cache.key_cache_sp[:1]]
                if comp is not None else [])
        res["runs"].append({
            "batch": B,
            "compressed_tokens_per_s": rnd(rc["tokens_per_s"], 1),
            "dense_tokens_per_s": rnd(rd["tokens_per_s"], 1),
            "compressed_decode_tokens_per_s": rnd(rc["decode_tokens_per_s"], 1),
            "dense_decode_tokens_per_s": rnd(rd["decode_tokens_per_s"], 1),
            "dense_sdpa_tokens_per_s": rnd(rs["tokens_per_s"], 1),
            "dense_sdpa_decode_tokens_per_s": rnd(rs["decode_tokens_per_s"], 1),
            "compressed_prefill_s": rnd(rc["prefill_s"], 4),
            "dense_prefill_s": rnd(rd["prefill_s"], 4),
            "compressed_kv_bytes": rc["kv_bytes"],
            "dense_kv_bytes": rd["kv_bytes"],
            "mean_retained_dims_layer0_k": lens[0] if lens else None,
            "same_tokens_frac": (round(float((rc["tokens"] == rd["tokens"]).float().mean()), 3)
                                 if comp is not None and dense is not None else None),
        })
    del comp, dense, sdpa, model
    torch.cuda.empty_cache()
    return res


def load_traffic(workload):
    """HBM bytes per split-kernel launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
    of this script (scaled by a plain copy of known size), as committed under profiles/; used
    only when it was measured on the library version that is loaded now."""
    from dynakv_amd import _lib

    path = os.path.join(ROOT, "profiles", f"splitk_{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    if t.get("dkv_version") != _lib.load().dkv_version():
        return None
    return {"bytes_per_launch": t["bytes_per_launch"], "source": os.path.relpath(path, ROOT)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prewarm-seconds", type=float, default=0.5,
                    help="untimed repeats of the first warmup step's attention launches (wall "
                         "seconds) so the timed steps run at sustained GPU clocks; 0 = none")
    ap.add_argument("--workload", default="config3", choices=["config3", "config2"])
    ap.add_argument("--layers", type=int, default=4,
                    help="independent layer caches per decode step (4 x ~190 MB at config 3)")
    ap.add_argument("--cpu-baseline-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-cutoff", action="store_true", help="skip the cutoff-head timing")
    ap.add_argument("--no-dense", action="store_true",
                    help="skip the dense (uncompressed) attention timing at the main shape")
    ap.add_argument("--no-config2", action="store_true",
                    help="skip the config-2 timing (fp16, B=4, 480 -> 580 tokens, one layer)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill-attention timing")
    ap.add_argument("--no-joint", action="store_true",
                    help="skip the joint-layout (rank 1024) attention timing")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip config 5 (greedy generation with a random Llama-3-8B, compressed "
                         "against uncompressed cache; about 10 s)")
    ap.add_argument("--e2e-only", action="store_true",
                    help="run config 5 alone (for a kernel trace of the decoder) and print its "
                         "JSON object")
    ap.add_argument("--e2e-batches", default="1,2,4", help="config 5 batch sizes")
    ap.add_argument("--e2e-long", default="16x8192",
                    help="batch x prompt of the long-context e2e run (compressed and dense "
                         "models, 50 new tokens), reported as e2e_long; 'none' to skip")
    ap.add_argument("--e2e-model", default="all", choices=["all", "compressed", "dense", "sdpa"],
                    help="config 5 models to run (one alone for a kernel trace of it)")
    ap.add_argument("--e2e-tokens", type=int, default=100, help="config 5 new tokens")
    ap.add_argument("--e2e-prompt", type=int, default=2048, help="config 5 prompt length")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (see the sharding "
              "design); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    e2e_batches = tuple(int(b) for b in args.e2e_batches.split(","))
    if args.e2e_only:
        print(json.dumps({"e2e": bench_e2e(dev, batches=e2e_batches, new_tokens=args.e2e_tokens,
                                           models=args.e2e_model,
                                           prompt_len=args.e2e_prompt)}),
              flush=True)
        return
    cfg = Config3 if args.workload == "config3" else Config2
    if args.copy_probe_mib > 0:
        # a plain device copy of known size: the reference point that scales the FETCH_SIZE and
        # WRITE_SIZE counters of a rocprofv3 --pmc run of this command
        nb = args.copy_probe_mib << 20
        src = torch.ones(nb, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize(dev)
        dst.copy_(src)
        torch.cuda.synchronize(dev)
        _log(f"copy probe: {args.copy_probe_mib} MiB read + {args.copy_probe_mib} MiB written")
        del src, dst
    r = run_gpu(cfg, args.steps, args.warmup, dev, args.layers, prewarm_s=args.prewarm_seconds)
    attn_s = r["attn_ms"] / 1e3
    gbs = r["bytes_total"] / attn_s / 1e9
    calls = r["calls"]
    split_avg_s = r["split_ms"] / 1e3 / calls
    # the split kernel merges its own splits (one launch per call) unless a merge kernel ran
    launch_bytes = r["bytes_per_call"] if r["merged_in_split"] else r["split_bytes_per_call"]
    achieved = launch_bytes / split_avg_s / 1e9
    layer_step_s = attn_s / calls
    traffic = load_traffic(cfg.name)
    dt_name = "bf16" if cfg.dtype == torch.bfloat16 else "fp16"
    # KernelPolicy(switch_tokens=500): the fused route below 500 tokens, two-stage from 500 on
    if cfg.S0 >= 500:
        route_label = "long_two_stage"
    elif r["final_len"] < 500:
        route_label = "short_fused"
    else:
        route_label = "short_fused below 500 tokens, long_two_stage from 500 (router)"
    line = {
        "metric": "decode-attn GB/s (% HBM peak) + decode tokens/s, Llama-3-8B shape, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_s"] * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp16",
        "data": "synthetic (seeded, generated on device; random orthogonal per-group bases)",
        "config": {
            "workload": cfg.name,
            "batch": cfg.B, "q_heads": cfg.Hq, "kv_heads": cfg.G, "head_dim": cfg.Dh,
            "rank": cfg.R, "cache_len_start": cfg.S0, "cache_len_end": r["final_len"],
            "mean_retention": cfg.mean, "route": route_label,
            "layout": "per-head (G=8, R=128)",
        },
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "layers_per_step": args.layers,
        # untimed: the first warmup step's attention launches repeated before the other warmup
        # steps (from idle the same launches run ~20% slower over the first ~100 ms of load)
        "prewarm_s": args.prewarm_seconds,
        "prewarm_launches": r["prewarm_calls"],
        "decode_attn_us_per_layer_step": round(layer_step_s * 1e6, 3),
        # a Llama-3-8B decode step runs 32 such layers: attention-only tokens/s of that stack
        "decode_tokens_per_s_attention_only_32_layers": round(cfg.B / (32 * layer_step_s), 1),
        "decode_tokens_per_s_step_wall": round(cfg.B * args.steps / r["wall_s"], 1),
        "host_syncs_total": r["syncs"],
        "roofline": {
            "kernel": f"splitk_kernel<{dt_name}, {'two_stage' if cfg.S0 >= 500 else 'fused / two_stage'}>",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes_per_launch"] if traffic else None,
            "split_kernel_us": round(r["split_ms"] * 1e3 / calls, 3),
            "timing": (f"HIP events around each step's {args.layers} back-to-back attention "
                       f"launches on their stream; per-launch time = that time / {args.layers}"),
            "algorithmic_bytes_per_launch": round(launch_bytes),
            "traffic_source": traffic["source"] if traffic else None,
        },
    }
    if not args.no_dense and cfg.name == "config3":
        _log("dense baseline attention at the same shape")
        line["dense_same_shape"] = bench_dense_same_shape(dev, S=r["final_len"],
                                                          prewarm_s=args.prewarm_seconds)
        line["dense_same_shape"]["compressed_split_kernel_us"] = line["roofline"]["split_kernel_us"]
    if not args.no_config2 and cfg.name == "config3":
        _log("config 2 (one layer, 480 -> 580 tokens)")
        line["config2"] = bench_config2(dev, prewarm_s=args.prewarm_seconds)
    if not args.no_cutoff:
        _log("cutoff head")
        line["cutoff_head"] = bench_cutoff(cfg, dev)
    if not args.no_joint:
        _log("joint layout")
        line["joint_layout"] = bench_joint(dev)
    if not args.no_prefill:
        _log("prefill attention")
        line["prefill_attention"] = bench_prefill(dev)
    if not args.no_e2e:
        _log("end-to-end generation (config 5)")
        line["e2e"] = bench_e2e(dev, batches=e2e_batches, new_tokens=args.e2e_tokens)
        if args.e2e_long != "none":
            lb, lp = (int(v) for v in args.e2e_long.lower().split("x"))
            _log(f"end-to-end generation, long context (batch {lb}, prompt {lp})")
            # the regime of the main workload: a cache large enough that the attention's bytes
            # count; the compressed cache holds half the dense cache's bytes
            line["e2e_long"] = bench_e2e(dev, batches=(lb,), prompt_len=lp, new_tokens=50,
                                         models="compressed,dense")
    if not args.no_cpu_baseline:
        _log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(cfg, r["workload"], r["cache"], args.cpu_baseline_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
