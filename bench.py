#!/usr/bin/env python3
# SPDX-License-Identifier: Apache-2.0
"""Benchmark of the routed-expert MoE layer out of MXFP4 on one MI355X.

A step is one pass of the layer over one batch of 64 synthetic decode tokens: router
(384 experts, top-8, fp64 logits, libm-exact sigmoid), expert-major gather, fused
gate/up + SiLU on the matrix cores, down projection, weighted combine in slot order.
All inputs are resident in HBM before the timed region (4 token batches rotated; the
8.98 GB expert bank is far larger than the last-level cache).

Also measured (extra keys of the same JSON line): the same layer at batch 1, and the
single 2048x7168 MXFP4 GEMV rotating over >= 1 GB of weight copies. Per-kernel times come
from HIP events the library records between its own launches (k3d_prof_*), on the
stream the kernels run on.

usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu]
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kimi-k3-in-c_amd"))

import k3amd  # noqa: E402
import workloads as wl  # noqa: E402

PEAK_HBM_GBS = 8000.0
PEAK_BF16_FLOPS = 2.5e15
E, I, N, K = wl.HIDDEN, wl.INTER, wl.N_EXPERTS, wl.TOPK
MAT_BYTES = I * E // 2 + I * E // 32          # one 2048x7168 MXFP4 matrix: 7,798,784 B
EXPERT_BYTES = 3 * MAT_BYTES                   # 23,396,352 B
ROUTER_BYTES = N * E * 4


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Layer:
    """The 384-expert layer resident on the device, the bank in the tiled layout."""

    def __init__(self, layout=k3amd.K3D_LAYOUT_TILED):
        L = k3amd.lib()
        k3amd.check(L.k3d_init(), "k3d_init")
        t0 = time.time()

        class Lazy:                     # experts generated one at a time while uploading
            def __len__(self):
                return N

            def __iter__(self):
                for e in range(N):
                    if e % 64 == 63:
                        log(f"bench: expert bank {e + 1}/{N} resident ({time.time() - t0:.1f} s)")
                    yield wl.expert(e)

        self.layout = layout
        self.bank = k3amd.DevBank(Lazy(), E, I, layout)
        self.router = k3amd.DevBuf(ROUTER_BYTES).upload(wl.router_weights())

    def free(self):
        self.bank.free()
        self.router.free()

    def run(self, x, out, idx, wt, T, ws, prec=0, stream=None, bias=None):
        k3amd.check(k3amd.lib().k3d_moe_routed(
            out.ptr, idx.ptr, wt.ptr, x.ptr, T, self.router.ptr, bias, self.bank.table.ptr,
            self.layout, E, I, N, K, 1, 1.0, k3amd.K3_ACT_SILU, 4.0, 25.0, prec, ws.ptr, ws.nbytes,
            None, None, None, stream), "k3d_moe_routed")


def time_layer(layer, T, steps, warmup, nbatch=4):
    L = k3amd.lib()
    xs = [k3amd.DevBuf(T * E * 4).upload(wl.tokens(T, tag=f"bench.tokens.{b}")) for b in range(nbatch)]
    out = k3amd.DevBuf(T * E * 4)
    idx = k3amd.DevBuf(T * K * 4)
    wt = k3amd.DevBuf(T * K * 4)
    ws = k3amd.DevBuf(L.k3d_moe_ws(T, E, I, N, K, 0))
    uniq = []
    for b in range(nbatch):                       # routing of each batch (outside timing)
        layer.run(xs[b], out, idx, wt, T, ws)
        h = idx.download(np.empty((T, K), np.int32))
        uniq.append(len(np.unique(h)))
    # HIP graphs of the whole layer: one replays it on all nbatch token batches in turn
    # (nbatch steps per launch, as a serving loop replays a decode step's layers from one
    # graph), one per batch covers the steps left over; step s runs batch s % nbatch
    stream = L.k3d_stream_create()
    if not stream:
        raise RuntimeError("k3d_stream_create: " + L.k3d_error().decode())

    def capture(batches):
        k3amd.check(L.k3d_graph_begin(stream), "k3d_graph_begin")
        for b in batches:
            layer.run(xs[b], out, idx, wt, T, ws, stream=stream)
        ex = C.c_void_p()
        k3amd.check(L.k3d_graph_end(stream, C.byref(ex)), "k3d_graph_end")
        return ex

    group = capture(range(nbatch))
    singles = [capture([b]) for b in range(nbatch)]

    def run_steps(n):
        for _ in range(n // nbatch):
            k3amd.check(L.k3d_graph_launch(group, stream), "k3d_graph_launch")
        for s in range(n % nbatch):
            k3amd.check(L.k3d_graph_launch(singles[s], stream), "k3d_graph_launch")

    run_steps(warmup)
    k3amd.check(L.k3d_sync(stream))
    t0 = time.perf_counter()                      # timed steps: graph replays, no profiler
    run_steps(steps)
    k3amd.check(L.k3d_sync(stream))
    t1 = time.perf_counter()
    for g in [group] + singles:
        L.k3d_graph_destroy(g)
    L.k3d_stream_destroy(stream)
    nprof = min(steps, 20)                        # stage breakdown: a separate profiled run
    prof = k3amd.Profile(max_marks=16 * nprof + 64)
    for s in range(nprof):
        layer.run(xs[s % nbatch], out, idx, wt, T, ws)
    k3amd.check(L.k3d_sync(None))
    stages = prof.end()
    for b in xs + [out, idx, wt, ws]:
        b.free()
    u_mean = float(np.mean([uniq[s % nbatch] for s in range(steps)]))
    return (t1 - t0), stages, u_mean, uniq


def time_prefill(layer, T=4096, steps=5, warmup=3, prof_reps=3):
    """Prefill layer (config 3): T tokens, bf16 activations, 96-token expert passes on the
    matrix cores. Eager calls after `warmup` untimed ones (the expert kernels take a few
    calls to reach their steady duration: the first timed call of a fresh process runs about
    15 % longer); the stage profile is the mean over prof_reps more calls."""
    L = k3amd.lib()
    x = k3amd.DevBuf(T * E * 4).upload(wl.tokens(T, tag="bench.prefill"))
    out = k3amd.DevBuf(T * E * 4)
    idx = k3amd.DevBuf(T * K * 4)
    wt = k3amd.DevBuf(T * K * 4)
    ws = k3amd.DevBuf(L.k3d_moe_ws(T, E, I, N, K, 1))
    for _ in range(warmup):
        layer.run(x, out, idx, wt, T, ws, prec=1)
    k3amd.check(L.k3d_sync(None))
    t0 = time.perf_counter()
    for _ in range(steps):
        layer.run(x, out, idx, wt, T, ws, prec=1)
    k3amd.check(L.k3d_sync(None))
    t1 = time.perf_counter()
    prof = k3amd.Profile(max_marks=16 * prof_reps)
    for _ in range(prof_reps):
        layer.run(x, out, idx, wt, T, ws, prec=1)
    k3amd.check(L.k3d_sync(None))
    st = prof.end()
    h = idx.download(np.empty((T, K), np.int32))
    for b in (x, out, idx, wt, ws):
        b.free()
    ms = (t1 - t0) / steps * 1e3
    flops = T * K * 3 * 2 * E * I                  # 2.886 TFLOP at T=4096
    expert_ms = sum(st.get(k, (0.0, 0))[0] / max(st.get(k, (0.0, 1))[1], 1) for k in ("gateup", "down"))
    return {"tokens": T, "ms_per_step": round(ms, 3), "tokens_per_s": round(T / ms * 1e3, 1),
            "arithmetic": "activations rounded to bf16 (one term), weights dequantized exactly, "
                          "bf16 MFMA with fp32 accumulation; tolerance 2e-2 relative",
            "expert_flops": flops, "expert_ms": round(expert_ms, 3),
            "expert_TFLOPs": round(flops / (expert_ms * 1e-3) / 1e12, 1) if expert_ms else None,
            "mfma_frac_of_bf16_peak": round(flops / (expert_ms * 1e-3) / 2.5e15, 4) if expert_ms else None,
            "unique_experts": int(len(np.unique(h))),
            "stages_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in st.items()}}


def time_expert_ffn(layer, per_graph=16, reps=20):
    """One routed expert SwiGLU FFN at decode (config 1): one token, gate/up/down out of the
    resident tiled bank, combine weight 0.125, through k3d_moe_experts with one assignment
    (the decode path). A HIP graph holds per_graph calls on per_graph different experts; the
    graph is replayed reps times, each replay on the next experts, so weights come from HBM."""
    L = k3amd.lib()
    x = k3amd.DevBuf(E * 4).upload(wl.expert_input())
    out = k3amd.DevBuf(E * 4)
    ids = np.arange(N, dtype=np.int32)
    idx = k3amd.DevBuf(N * 4).upload(ids)
    wt = k3amd.DevBuf(4).upload(np.array([0.125], np.float32))
    ws = k3amd.DevBuf(L.k3d_moe_ws(1, E, I, N, 1, 0))
    stream = L.k3d_stream_create()
    ngraph = N // per_graph
    graphs = []
    for gi in range(ngraph):
        k3amd.check(L.k3d_graph_begin(stream), "k3d_graph_begin")
        for c in range(per_graph):
            e = gi * per_graph + c
            k3amd.check(L.k3d_moe_experts(out.ptr, idx.ptr + 4 * e, wt.ptr, x.ptr, 1, layer.bank.table.ptr,
                                          layer.layout, E, I, N, 1, k3amd.K3_ACT_SILU, 4.0, 25.0, 0,
                                          ws.ptr, ws.nbytes, None, None, None, stream), "k3d_moe_experts")
        ex = C.c_void_p()
        k3amd.check(L.k3d_graph_end(stream, C.byref(ex)), "k3d_graph_end")
        graphs.append(ex)
    for g in graphs[:2]:
        k3amd.check(L.k3d_graph_launch(g, stream), "k3d_graph_launch")
    k3amd.check(L.k3d_sync(stream))
    t0 = time.perf_counter()
    for r in range(reps):
        k3amd.check(L.k3d_graph_launch(graphs[r % ngraph], stream), "k3d_graph_launch")
    k3amd.check(L.k3d_sync(stream))
    t1 = time.perf_counter()
    for g in graphs:
        L.k3d_graph_destroy(g)
    L.k3d_stream_destroy(stream)
    for b in (x, out, idx, wt, ws):
        b.free()
    us = (t1 - t0) / (reps * per_graph) * 1e6
    algo = EXPERT_BYTES + 2 * E * 4
    return {"tokens": 1, "experts_rotated": N, "us_per_call": round(us, 2),
            "tokens_per_s": round(1e6 / us, 1), "algorithmic_bytes": algo,
            "GBps": round(algo / (us * 1e-6) / 1e9, 1),
            "frac_of_peak": round(algo / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}


def time_skewed(layer, T=512, steps=5, warmup=3, prof_reps=3):
    """Skewed routing + dense trunk (config 4): T tokens, router selection bias giving
    Zipf(1.2)-like expert popularity, routed experts with bf16 activations, then the
    always-on bf16 shared expert (7168 -> 2048 -> 7168) accumulated onto the output."""
    L = k3amd.lib()
    x = k3amd.DevBuf(T * E * 4).upload(wl.tokens(T, tag="bench.skewed"))
    bias = k3amd.DevBuf(N * 4).upload(wl.zipf_bias())
    w1, w3, w2 = wl.shared_expert_weights()
    d1, d3, d2 = (k3amd.DevBuf(w.nbytes).upload(w) for w in (w1, w3, w2))
    out = k3amd.DevBuf(T * E * 4)
    idx = k3amd.DevBuf(T * K * 4)
    wt = k3amd.DevBuf(T * K * 4)
    ws = k3amd.DevBuf(L.k3d_moe_ws(T, E, I, N, K, 1))
    sws_b = L.k3d_shared_ws(T, E, I, 1)
    sws = k3amd.DevBuf(sws_b)

    def step():
        layer.run(x, out, idx, wt, T, ws, prec=1, bias=bias.ptr)
        k3amd.check(L.k3d_shared_expert(out.ptr, 1, x.ptr, T, d1.ptr, d3.ptr, d2.ptr, E, I,
                                        k3amd.K3_ACT_SILU, 4.0, 25.0, 1, sws.ptr, sws_b, None),
                    "k3d_shared_expert")
    for _ in range(warmup):
        step()
    k3amd.check(L.k3d_sync(None))
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    k3amd.check(L.k3d_sync(None))
    t1 = time.perf_counter()
    prof = k3amd.Profile(max_marks=16 * prof_reps)
    for _ in range(prof_reps):
        step()
    k3amd.check(L.k3d_sync(None))
    st = prof.end()
    # one more step with per-workgroup stamps of the routed expert kernels
    sbuf = k3amd.DevBuf(1 << 20)
    k3amd.check(L.k3d_stamps_begin(sbuf.ptr, sbuf.nbytes), "k3d_stamps_begin")
    step()
    k3amd.check(L.k3d_sync(None))
    kinds, grids = (C.c_int * 64)(), (C.c_int * 64)()
    nst = C.c_int()
    k3amd.check(L.k3d_stamps_end(kinds, grids, 64, C.byref(nst)), "k3d_stamps_end")
    nwg = sum(grids[i] for i in range(min(nst.value, 64)))
    stamps = sbuf.download(np.empty((nwg, 3), np.uint64))
    sbuf.free()
    h = idx.download(np.empty((T, K), np.int32))
    for b in (x, bias, d1, d3, d2, out, idx, wt, ws, sws):
        b.free()
    cnt = np.sort(np.bincount(h.ravel(), minlength=N))[::-1]
    ms = (t1 - t0) / steps * 1e3
    mean = lambda k: st.get(k, (0.0, 1))[0] / max(st.get(k, (0.0, 1))[1], 1)
    sh_ms = mean("shared")
    sh_flops = T * 3 * 2 * E * I
    routed_ms = mean("gateup") + mean("down")
    u = int((cnt > 0).sum())
    routed_bytes = u * EXPERT_BYTES
    routed_flops = T * K * 3 * 2 * E * I
    bound_ms = max(routed_bytes / (PEAK_HBM_GBS * 1e9), routed_flops / PEAK_BF16_FLOPS) * 1e3
    step_bytes = routed_bytes + 3 * I * E * 2 + ROUTER_BYTES + 2 * T * E * 4
    step_flops = routed_flops + sh_flops
    step_bound_ms = max(step_bytes / (PEAK_HBM_GBS * 1e9), step_flops / PEAK_BF16_FLOPS) * 1e3
    return {"tokens": T, "ms_per_step": round(ms, 3), "tokens_per_s": round(T / ms * 1e3, 1),
            "arithmetic": "routed and shared experts with activations rounded to bf16 (one term), "
                          "bf16 MFMA with fp32 accumulation; tolerance 2e-2 relative",
            "skew": "selection bias 2.5 * rank^-1.2 over a seeded expert permutation (the form of "
                    "the reference's e_score_correction_bias: it steers which experts are chosen, "
                    "the combine weights stay the unbiased scores); with top-8 of distinct experts "
                    "no expert can hold more than 1/8 of the assignments, so Zipf(1.2)'s top-3 "
                    "share of 41.8 % is capped at 37.5 %",
            "roofline": {"bound": "max(hbm, mfma)",
                         "routed_stage_ms": round(routed_ms, 4),
                         "routed_bound_ms": round(bound_ms, 4),
                         "routed_frac": round(bound_ms / routed_ms, 4) if routed_ms else None,
                         "routed_bytes": routed_bytes, "routed_flops": routed_flops,
                         "step_bound_ms": round(step_bound_ms, 4),
                         "step_frac": round(step_bound_ms / ms, 4)},
            "per_cu_busy": cu_busy(stamps),
            "routing": {"unique_experts": u, "max_tokens_per_expert": int(cnt[0]),
                        "mean_tokens_per_used_expert": round(float(cnt[cnt > 0].mean()), 2),
                        "share_top1": round(float(cnt[0] / cnt.sum()), 4),
                        "share_top3": round(float(cnt[:3].sum() / cnt.sum()), 4),
                        "share_top8": round(float(cnt[:8].sum() / cnt.sum()), 4),
                        "histogram_top16": [int(v) for v in cnt[:16]]},
            "shared_expert_ms": round(sh_ms, 4),
            "shared_expert_TFLOPs": round(sh_flops / (sh_ms * 1e-3) / 1e12, 1) if sh_ms else None,
            "stages_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in st.items()}}


def cu_busy(stamps):
    """Per-CU busy time of the stamped expert launches of one step (k3d_stamps_*): a CU is
    busy while any of its workgroups runs (the union of their [start, end] intervals on the
    100 MHz clock), over all launches of the step; min / median / max over the CUs that
    ran one, beside the span from the first start to the last end."""
    if len(stamps) == 0:
        return None
    t0, t1, hw = stamps[:, 0].astype(np.int64), stamps[:, 1].astype(np.int64), stamps[:, 2]
    xcc = (hw >> np.uint64(32)).astype(np.int64)
    hid = (hw & np.uint64(0xFFFFFFFF)).astype(np.int64)
    key = xcc * 256 + ((hid >> 8) & 0xFF)             # XCC, shader engine / array, CU
    busy = []
    for k in np.unique(key):
        sel = np.argsort(t0[key == k])
        a, b = t0[key == k][sel], t1[key == k][sel]
        tot, cs, ce = 0, a[0], b[0]
        for s_, e_ in zip(a[1:], b[1:]):
            if s_ > ce:
                tot += ce - cs
                cs, ce = s_, e_
            else:
                ce = max(ce, e_)
        busy.append((tot + ce - cs) / 100.0)           # 100 MHz ticks -> us
    busy = np.array(busy)
    span = (t1.max() - t0.min()) / 100.0
    return {"cus": int(len(busy)), "workgroups": int(len(stamps)), "span_us": round(float(span), 1),
            "busy_us": {"min": round(float(busy.min()), 1), "median": round(float(np.median(busy)), 1),
                        "max": round(float(busy.max()), 1)},
            "busy_frac_of_span": {"min": round(float(busy.min() / span), 3),
                                  "median": round(float(np.median(busy) / span), 3)}}


def time_k3_moe(T=1, steps=20, n_experts=896, distinct=32):
    """Kimi K3's MoE layer at its real shape through the reference-compatible k3_moe
    (hidden 7168, latent 3584, moe_inter 3072, 896 experts, top-16 with a selection bias,
    two shared experts, bf16 trunk: router, down-projection, routed experts, latent RMSNorm,
    up-projection, shared expert), the routed experts served from the library's HBM bank
    behind K3ExpertSrc (896 slots of 17,547,264 B, 15.7 GB; `distinct` generated experts
    placed under all 896 ids, each slot its own copy in HBM) and the trunk weights
    registered resident. Wall clock per call of T tokens, including the copy of x to the
    device and of out back; tokens rotate over 8 batches."""
    L = k3amd.lib()
    cfg, W, ex = wl.latent_layer(E, 3584, 3072, n_experts, 16, tag="bench.k3", n_generated=distinct)
    runs = [wl.expert_run(ex[e]) for e in range(distinct)]
    bank = k3amd.HbmBank(1, n_experts, 3584, 3072, n_experts, k3amd.K3D_LAYOUT_TILED, None)
    try:
        for e in range(n_experts):
            bank.put_run(0, e, runs[e % distinct])
        for k in ("gate", "bias", "latent_norm", "down", "up", "sh1", "sh3", "sh2"):
            k3amd.dev_register(W[k])
        xs = [wl.tokens(T, E, tag=f"bench.k3.x.{b}") for b in range(8)]
        for b in range(3):
            k3amd.moe(xs[b], cfg, W, 1, bank.src, 0 if T == 1 else 1)
        st0 = bank.stats()
        t0 = time.perf_counter()
        for i in range(steps):
            k3amd.moe(xs[i % 8], cfg, W, 1, bank.src, 0 if T == 1 else 1)
        t1 = time.perf_counter()
        moved = bank.stats()["bytes_uploaded"] - st0["bytes_uploaded"]
        for k in ("gate", "bias", "latent_norm", "down", "up", "sh1", "sh3", "sh2"):
            L.k3_dev_unregister(W[k].ctypes.data)
    finally:
        bank.destroy()
    ms = (t1 - t0) / steps * 1e3
    return {"entry": "k3_moe" if T == 1 else "k3_moe_prefill", "tokens": T, "hidden": E,
            "latent": 3584, "moe_inter": 3072, "experts": n_experts, "topk": 16, "n_shared": 2,
            "trunk": "bf16", "ms_per_call": round(ms, 3), "tokens_per_s": round(T / ms * 1e3, 1),
            "bank_GB": round(n_experts * 17547264 / 1e9, 2), "weight_bytes_uploaded_while_timed": int(moved)}


def time_back_to_back(launch, ncalls, per_graph=64, reps=8):
    """Wall-clock microseconds per call of `launch(i, stream)` run back to back: per_graph
    consecutive calls captured in one HIP graph, the graph replayed reps times (calls
    i = 0, 1, ... across the whole run, ncalls distinct), no events between launches."""
    L = k3amd.lib()
    stream = L.k3d_stream_create()
    ngraph = max(1, ncalls // per_graph)
    graphs = []
    for g in range(ngraph):
        k3amd.check(L.k3d_graph_begin(stream), "k3d_graph_begin")
        for c in range(per_graph):
            launch(g * per_graph + c, stream)
        ex = C.c_void_p()
        k3amd.check(L.k3d_graph_end(stream, C.byref(ex)), "k3d_graph_end")
        graphs.append(ex)
    for g in graphs:
        k3amd.check(L.k3d_graph_launch(g, stream), "k3d_graph_launch")
    k3amd.check(L.k3d_sync(stream))
    t0 = time.perf_counter()
    for r in range(reps):
        k3amd.check(L.k3d_graph_launch(graphs[r % ngraph], stream), "k3d_graph_launch")
    k3amd.check(L.k3d_sync(stream))
    t1 = time.perf_counter()
    for g in graphs:
        L.k3d_graph_destroy(g)
    L.k3d_stream_destroy(stream)
    return (t1 - t0) / (reps * per_graph) * 1e6


def time_gemv(steps=200, copies=128, rows=2048, inn=E, scale_byte=None):
    """rows x inn MXFP4 GEMV, one token, rotating over `copies` distinct weight copies
    (>= 1 GB, well past the last-level cache) so every launch streams from HBM. Kernel time
    from HIP events around each launch; throughput from back-to-back launches in a graph.
    scale_byte: every E8M0 byte that value (the reference kernel benchmark's 127) instead of
    the configured distribution."""
    L = k3amd.lib()
    packed, scales, x = wl.gemv_inputs(rows, inn)
    if scale_byte is not None:
        scales = np.full_like(scales, scale_byte)
    pk_b, sc_b = packed.nbytes, scales.nbytes
    stride = (pk_b + sc_b + 4095) // 4096 * 4096
    w = k3amd.DevBuf(copies * stride)
    w.upload(packed, 0).upload(scales, pk_b)
    for c in range(1, copies):
        k3amd.check(L.k3d_h2d(w.ptr + c * stride, packed.ctypes.data, pk_b, None))
        k3amd.check(L.k3d_h2d(w.ptr + c * stride + pk_b, scales.ctypes.data, sc_b, None))
    k3amd.check(L.k3d_sync(None))
    dx = k3amd.DevBuf(inn * 4).upload(x)
    dy = k3amd.DevBuf(rows * 4)
    ws = k3amd.DevBuf(L.k3d_matmul_mxfp4_ws(1, inn))

    def launch(c, stream=None):
        base = w.ptr + (c % copies) * stride
        k3amd.check(L.k3d_matmul_mxfp4(dy.ptr, dx.ptr, 1, base, base + pk_b, inn, rows, 0, ws.ptr,
                                       ws.nbytes, stream), "k3d_matmul_mxfp4")
    for c in range(20):
        launch(c)
    k3amd.check(L.k3d_sync(None))
    prof = k3amd.Profile(max_marks=4 * steps + 16)
    for c in range(steps):
        launch(c)
    k3amd.check(L.k3d_sync(None))
    st = prof.end()
    b2b = time_back_to_back(launch, copies)
    for b in (w, dx, dy, ws):
        b.free()
    algo = pk_b + sc_b + inn * 4 + rows * 4        # weights + x + y (7,835,648 B at 2048 x 7168)
    ms, n = st.get("gemv", (0.0, 0))
    kern_ms = ms / max(n, 1)
    return {"shape": [rows, inn], "copies_rotated": copies, "algorithmic_bytes": algo,
            "kernel_us": round(kern_ms * 1e3, 3),
            "kernel_GBps": round(algo / (kern_ms * 1e-3) / 1e9, 1),
            "frac_of_peak": round(algo / (kern_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "back_to_back_us": round(b2b, 3),
            "back_to_back_frac_of_peak": round(algo / (b2b * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}


def time_trunk_gemv(rows=12288, inn=7168, copies=4, steps=40):
    """The bf16 trunk GEMV of the reference's kernel benchmark (KDA q-projection, 7168 ->
    12288, benchmarks/bench_kernels.c:102-127) through k3d_matmul_bf16, one token, over
    `copies` weight copies (704 MB, past the 256 MB last-level cache)."""
    L = k3amd.lib()
    Wb = k3amd.gen_bf16_normal(rows * inn, wl.stream("trunk.w"), 0.0, 0.02)
    x = k3amd.gen_normal(inn, wl.stream("trunk.x"))
    stride = (Wb.nbytes + 4095) // 4096 * 4096
    w = k3amd.DevBuf(copies * stride)
    for c in range(copies):
        w.upload(Wb, c * stride)
    dx = k3amd.DevBuf(inn * 4).upload(x)
    dy = k3amd.DevBuf(rows * 4)

    def launch(c, stream=None):
        k3amd.check(L.k3d_matmul_bf16(dy.ptr, dx.ptr, 1, w.ptr + (c % copies) * stride, inn, rows,
                                      stream), "k3d_matmul_bf16")
    for c in range(8):
        launch(c)
    k3amd.check(L.k3d_sync(None))
    prof = k3amd.Profile(max_marks=4 * steps + 16)
    for c in range(steps):
        launch(c)
    k3amd.check(L.k3d_sync(None))
    st = prof.end()
    b2b = time_back_to_back(launch, 4 * copies, per_graph=16)
    for b in (w, dx, dy):
        b.free()
    algo = rows * inn * 2 + inn * 4 + rows * 4
    ms, n = st.get("gemv", (0.0, 0))
    kern_ms = ms / max(n, 1)
    return {"shape": [rows, inn], "copies_rotated": copies, "algorithmic_bytes": algo,
            "kernel_us": round(kern_ms * 1e3, 3),
            "kernel_GBps": round(algo / (kern_ms * 1e-3) / 1e9, 1),
            "frac_of_peak": round(algo / (kern_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "back_to_back_us": round(b2b, 3)}


def cpu_baseline(T_sample=8, budget_s=10.0):
    """The reference's own kernels (oracle/_ref, compiled from its src/core/k3_ops.c) in
    the reference composition, on the host cores, over a bounded sample of the batch-64
    workload: the first T_sample tokens of batch 0. Runs in the process it is called in,
    with the OpenMP threads that process's environment sets."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, Ref
    kind = "reference" if Ref.available() else "port"
    impl = Ref() if kind == "reference" else Oracle()
    threads = Oracle().threads()
    W = wl.router_weights()
    X = wl.tokens(64, tag="bench.tokens.0")[:T_sample]
    idx = np.stack([impl.router(X[t], W, None, K)[0] for t in range(T_sample)])
    bank = wl.lazy_bank(idx)
    impl.moe_routed(X[:1], W, None, bank, E, I, K)          # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        impl.moe_routed(X, W, None, bank, E, I, K)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": round(T_sample / med, 3), "unit": "tokens/s", "cores": threads,
            "kind": kind,
            "sample": f"{T_sample} tokens of the batch-64 decode layer (router + 8 experts each, "
                      f"SiLU), {len(times)} reps after one warm-up, median; spread "
                      f"{min(times):.3f}-{max(times):.3f} s",
            "composition": "k3_router per token, then k3_moe's per-token routed loop (k3_ops.c:"
                           "576-643) with z := x: three k3_matmul_mxfp4 calls per (token, slot). "
                           "The reference's expert-major k3_moe_prefill chunk makes the same "
                           "per-(token, slot) GEMV calls (it has no batched MXFP4 kernel) and only "
                           "reorders them, reusing each expert about 1.8x at batch 64",
            "ms_per_token": round(med / T_sample * 1e3, 2)}


def host_cores():
    """(physical cores, logical CPUs) this process may run on: the CPUs of its affinity
    mask, grouped by (socket, core) from /proc/cpuinfo."""
    cpus = sorted(os.sched_getaffinity(0))
    core_of, cur = {}, {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if "processor" in cur:
                        core_of[cur["processor"]] = (cur.get("physical id", "0"),
                                                     cur.get("core id", cur["processor"]))
                    cur = {}
                    continue
                k, v = (t.strip() for t in line.split(":", 1))
                if k in ("processor", "physical id", "core id"):
                    cur[k] = v
        if "processor" in cur:
            core_of[cur["processor"]] = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
    except OSError:
        pass
    phys = {core_of.get(str(c), ("?", str(c))) for c in cpus}
    return len(phys), len(cpus)


def cpu_baseline_children():
    """The CPU baseline in child processes started before this process touches the GPU, so
    that the OpenMP runtime of each child starts with its own thread count: all physical
    cores of this process's CPU share (at most the OMP_NUM_THREADS the environment allows),
    then one thread, both with OMP_PROC_BIND=close and OMP_PLACES=cores."""
    import subprocess
    phys, logical = host_cores()
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    all_threads = max(1, min(phys, cap) if cap > 0 else phys)
    res = {}
    for label, n, sample in (("all", all_threads, 8), ("one", 1, 1)):
        env = dict(os.environ, OMP_NUM_THREADS=str(n), OMP_PROC_BIND="close", OMP_PLACES="cores")
        log(f"bench: CPU baseline on {n} thread(s) in a child process")
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", str(sample)],
                           env=env, capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError(f"CPU baseline child failed ({r.returncode}): {r.stderr[-2000:]}")
        res[label] = json.loads(r.stdout.strip().splitlines()[-1])
    out = res["all"]
    one = res["one"]
    out["one_thread"] = {"value": one["value"], "unit": one["unit"], "cores": one["cores"],
                         "sample": one["sample"], "ms_per_token": one["ms_per_token"]}
    out["host"] = host_description(phys, logical)
    out["env"] = "OMP_PROC_BIND=close OMP_PLACES=cores, OMP_NUM_THREADS set per child"
    return out


def host_description(phys=None, logical=None):
    """CPU model, core counts, AVX-512 presence and the C library version of the host the
    CPU numbers come from."""
    import platform
    model, avx512 = None, None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if model is None and line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                if avx512 is None and line.startswith("flags"):
                    avx512 = " avx512f " in f" {line.split(':', 1)[1].strip()} "
                if model is not None and avx512 is not None:
                    break
    except OSError:
        pass
    return {"cpu": model, "physical_cores": phys, "logical_cpus": logical,
            "avx512f": avx512, "isa_path": "the reference's AVX2+FMA intrinsic path",
            "libc": " ".join(platform.libc_ver())}


def measured_traffic():
    """HBM bytes per GATEUP dispatch at batch 64 from the profiler's byte counters (two
    counter passes over this bench, scaled by a copy of known size), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            return int(json.load(f)["traffic_bytes_per_dispatch"])
    except (OSError, KeyError, ValueError):
        return None


def copy_probe(nbytes=256 << 20, reps=10):
    """A plain device-to-device copy kernel of known size: reads and writes nbytes each."""
    import torch
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"bench: copy probe {reps} x {nbytes} B read + {nbytes} B written")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-child", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--only", nargs="+", default=None,
                    help="time only these workloads (decode64 batch1 gemv gemv_ref trunk ffn "
                         "prefill skewed k3moe k3moe64) and print their figures instead of the "
                         "benchmark line")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 256 MiB device copy 10 times (calibrates the HBM "
                         "byte counters of a profiler run) and exit")
    args = ap.parse_args()
    if args.cpu_child:
        print(json.dumps(cpu_baseline(T_sample=args.cpu_child, budget_s=10.0 if args.cpu_child > 1 else 3.0)))
        return
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build does not shard the layer across GPUs)", file=sys.stderr)
        sys.exit(2)

    if args.only:
        # a subset of the extra workloads, for kernel work: one JSON object, not the line
        res = {}
        need_layer = {"decode64", "batch1", "ffn", "prefill", "skewed"} & set(args.only)
        layer = Layer() if need_layer else None
        for name in args.only:
            if name == "decode64":
                secs, st, u, _ = time_layer(layer, 64, args.steps, args.warmup)
                res[name] = {"ms_per_step": round(secs / args.steps * 1e3, 4), "unique": u,
                             "stages_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in st.items()}}
            elif name == "batch1":
                n = max(args.steps * 5, 50)
                secs, st, u, _ = time_layer(layer, 1, n, args.warmup)
                res[name] = {"ms_per_step": round(secs / n * 1e3, 4),
                             "stages_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in st.items()}}
            elif name == "gemv":
                res[name] = time_gemv()
            elif name == "gemv_ref":
                res[name] = time_gemv(copies=192, rows=3072, inn=3584, scale_byte=127)
            elif name == "k3moe":
                res[name] = time_k3_moe(1)
            elif name == "k3moe64":
                res[name] = time_k3_moe(64, steps=5)
            elif name == "trunk":
                res[name] = time_trunk_gemv()
            elif name == "ffn":
                res[name] = time_expert_ffn(layer)
            elif name == "prefill":
                res[name] = time_prefill(layer)
            elif name == "skewed":
                res[name] = time_skewed(layer)
            else:
                raise SystemExit(f"unknown section {name}")
            log(f"bench: {name} {res[name]}")
        print(json.dumps(res), flush=True)
        return

    cb = None if args.no_cpu else cpu_baseline_children()    # before any GPU call
    layer = Layer()
    T = 64
    secs, stages, u_mean, uniq = time_layer(layer, T, args.steps, args.warmup)
    ms_step = secs / args.steps * 1e3
    tok_s = T * args.steps / secs
    layer_bytes = u_mean * EXPERT_BYTES + ROUTER_BYTES + 2 * T * E * 4
    gu_ms, gu_n = stages.get("gateup", (0.0, 1))
    gu_ms /= max(gu_n, 1)
    gu_bytes = u_mean * 2 * MAT_BYTES + T * E * 4 + T * K * I * 4
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9 if gu_ms > 0 else 0.0
    log(f"bench: batch-64 layer {ms_step:.3f} ms/step, {tok_s:.0f} tok/s; stages "
        + ", ".join(f"{k} {v[0] / max(v[1], 1):.3f} ms" for k, v in stages.items()))

    s1, st1, u1, _ = time_layer(layer, 1, max(args.steps * 5, 50), args.warmup)
    b1_ms = s1 / max(args.steps * 5, 50) * 1e3
    b1_bytes = u1 * EXPERT_BYTES + ROUTER_BYTES
    log(f"bench: batch-1 layer {b1_ms:.3f} ms/step")
    gemv = time_gemv()
    log(f"bench: gemv {gemv}")
    gemv_ref = time_gemv(copies=192, rows=3072, inn=3584, scale_byte=127)
    log(f"bench: gemv (reference benchmark shape) {gemv_ref}")
    trunk = time_trunk_gemv()
    log(f"bench: trunk gemv {trunk}")
    ffn = time_expert_ffn(layer)
    log(f"bench: expert ffn {ffn}")
    prefill = time_prefill(layer)
    log(f"bench: prefill {prefill}")
    skewed = time_skewed(layer)
    log(f"bench: skewed {skewed}")
    layer.free()
    k3moe = time_k3_moe(1)
    log(f"bench: k3_moe at the K3 shape {k3moe}")
    line = {
        "metric": "MoE-layer tokens/s + achieved HBM GB/s (MXFP4 expert GEMV), batch 1 & 64",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "compute": "MXFP4 weights dequantized exactly to bf16 in registers; activations as bf16 "
                   "hi+lo; MFMA with fp32 accumulation; fp64 router logits",
        "data": "synthetic",
        "timing": "the layer captured in HIP graphs: one replays it on the 4 token batches in turn "
                  "(4 steps per launch, as a serving loop replays a decode step's layers), per-batch "
                  "graphs for steps past a multiple of 4; batch 1 the same",
        "config": {"workload": "moe_decode_batch64", "tokens": T, "hidden": E, "inter": I,
                   "experts": N, "topk": K, "activation": "silu", "bank_GB": round(N * EXPERT_BYTES / 1e9, 3),
                   "unique_experts_per_step": round(u_mean, 1)},
        "roofline": {"bound": "hbm",
                     "kernel": "mx_moe_kernel GATEUP (fused gate/up + SiLU, tiled bank)",
                     "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "profiles/hbm_traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE "
                                       "passes over this bench, scaled by a copy kernel of known size",
                     "kernel_ms": round(gu_ms, 4), "algorithmic_bytes": int(gu_bytes)},
        "layer_GBps": round(layer_bytes / (ms_step * 1e-3) / 1e9, 1),
        "stages_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in stages.items()},
        "batch1": {"tokens_per_s": round(1e3 / b1_ms, 1), "ms_per_step": round(b1_ms, 4),
                   "layer_GBps": round(b1_bytes / (b1_ms * 1e-3) / 1e9, 1),
                   "stages_ms": {k: round(v[0] / max(v[1], 1), 4) for k, v in st1.items()}},
        "gemv_2048x7168": gemv,
        "gemv_3072x3584_refbench": dict(gemv_ref, inputs="the reference kernel benchmark's "
                                        "shape and scale bytes (all 127, bench_kernels.c:129-140); "
                                        "codes and x from the library's generator"),
        "trunk_gemv_bf16_12288x7168": trunk,
        "expert_ffn_decode": ffn,
        "prefill_4096": prefill,
        "skewed_512_shared": skewed,
        "k3_moe_decode_k3_shape": k3moe,
    }
    if cb is not None:
        line["cpu_baseline"] = cb
        line["gpu_over_cpu"] = round(tok_s / cb["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
