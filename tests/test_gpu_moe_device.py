# SPDX-License-Identifier: Apache-2.0
"""The device-resident MoE path (k3d_moe_routed) on both bank layouts: the tiled layout's
bytes, row-major vs tiled results bit-identical, parity with the oracle (routing and the
gather permutation bit-exact, outputs within 1e-4 * ||ref||inf; bf16 activations within
2e-2 relative), and the full decode shape against the reference's golden outputs."""
import sys

import numpy as np
import pytest

from conftest import max_err_rel_inf

pytestmark = pytest.mark.gpu
TOL = 1e-4
TOL_BF16 = 2e-2


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def tile_layout(packed, scales, rows, K):
    """The tiled layout, restated with numpy: rows padded to a multiple of 64, tiles of 16
    rows in groups of 4 (u = tile in group); in group q, chunk c (16 blocks), tile u, step d,
    lane l = 16g + r holds block 4d+g of row 64q+16u+r; its four scale bytes (d = 0..3) are
    contiguous at [((q*nchunk + c)*4 + u)*256 + 4l]. A block with scale byte 255 (NaN) is
    stored as zero codes with scale byte 127."""
    ngrp, nchunk, nblk = (rows + 63) // 64, K // 512, K // 32
    P = np.zeros((ngrp * 64, K // 2), np.uint8)
    S = np.zeros((ngrp * 64, nblk), np.uint8)
    P[:rows] = packed.reshape(rows, K // 2)
    S[:rows] = scales.reshape(rows, nblk)
    nan = S == 255
    P.reshape(ngrp * 64, nblk, 16)[nan] = 0
    S[nan] = 127
    Pb = P.reshape(ngrp, 4, 16, nchunk, 4, 4, 16)        # q, u, r, c, d, g, byte
    tp = Pb.transpose(0, 3, 1, 4, 5, 2, 6).reshape(-1)   # q, c, u, d, (g, r), byte
    Sb = S.reshape(ngrp, 4, 16, nchunk, 4, 4)            # q, u, r, c, d, g
    ts = Sb.transpose(0, 3, 1, 5, 2, 4).reshape(-1)      # q, c, u, (g, r), d
    return tp, ts


@pytest.mark.parametrize("rows,K", [(40, 1024), (16, 512), (2048, 7168)])
def test_tile_layout_bytes(gpu, rows, K):
    say(f"case: tile layout rows={rows} K={K}")
    L = gpu.lib()
    rng = np.random.default_rng(rows + K)
    packed = rng.integers(0, 256, rows * K // 2, dtype=np.uint8)
    scales = rng.integers(0, 256, rows * K // 32, dtype=np.uint8)
    import ctypes as C
    pk, sc = C.c_size_t(), C.c_size_t()
    gpu.check(L.k3d_mxfp4_tiled_size(rows, K, C.byref(pk), C.byref(sc)), "size")
    src_p = gpu.DevBuf(packed.nbytes).upload(packed)
    src_s = gpu.DevBuf(scales.nbytes).upload(scales)
    dst_p, dst_s = gpu.DevBuf(pk.value), gpu.DevBuf(sc.value)
    gpu.check(L.k3d_mxfp4_tile(dst_p.ptr, dst_s.ptr, src_p.ptr, src_s.ptr, rows, K, None), "tile")
    gpu.check(L.k3d_sync(None), "sync")
    got_p = dst_p.download(np.empty(pk.value, np.uint8))
    got_s = dst_s.download(np.empty(sc.value, np.uint8))
    for b in (src_p, src_s, dst_p, dst_s):
        b.free()
    tp, ts = tile_layout(packed, scales, rows, K)
    assert np.array_equal(got_p, tp)
    assert np.array_equal(got_s, ts)


def test_tile_rejects_bad_width(gpu):
    L = gpu.lib()
    assert L.k3d_mxfp4_tile(None, None, None, None, 16, 480, None) != 0
    assert b"512" in L.k3d_error()


def nan_scaled(k3, E, I, seed, e):
    """An expert whose gate and down matrices carry NaN (255) scale bytes: those blocks
    contribute zero (reference k3_ops.c mxfp4 paths)."""
    ex = k3.gen_expert(E, I, seed, e)
    t = [a.copy() for a in ex.t]
    t[1][5::37] = 255
    t[5][3::41] = 255
    return k3.Expert(*t)


@pytest.fixture(scope="module")
def small_layer(k3):
    E, I, N, K, T = 1024, 512, 16, 4, 29
    rng = np.random.default_rng(31)
    bank = [k3.gen_expert(E, I, 41, e) for e in range(N)]
    bank[3] = nan_scaled(k3, E, I, 41, 3)
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    return dict(E=E, I=I, N=N, K=K, T=T, bank=bank, W=W, bias=bias, X=X)


def stable_gather(idx, n_experts):
    a = idx.reshape(-1)
    perm = np.argsort(a, kind="stable").astype(np.int32)
    off = np.zeros(n_experts + 1, np.int32)
    np.cumsum(np.bincount(a, minlength=n_experts), out=off[1:])
    return perm, off


@pytest.mark.parametrize("prec", [0, 1])
def test_moe_device_layouts_vs_oracle(gpu, orc, small_layer, prec):
    s = small_layer
    say(f"case: device moe layouts prec={prec} E={s['E']} I={s['I']} T={s['T']}")
    res = {}
    for layout in (gpu.K3D_LAYOUT_ROWS, gpu.K3D_LAYOUT_TILED):
        bank = gpu.DevBank(s["bank"], s["E"], s["I"], layout)
        try:
            res[layout] = gpu.moe_routed_device(bank, s["X"], s["W"], s["bias"], s["K"], prec=prec,
                                                inter=s["I"])
        finally:
            bank.free()
    r, t = res[gpu.K3D_LAYOUT_ROWS], res[gpu.K3D_LAYOUT_TILED]
    for a, b in zip(r, t):
        assert np.array_equal(np.asarray(a), np.asarray(b))       # layouts: identical bits
    out, idx, wt, perm, off, drops = r
    o2, i2, w2 = orc.moe_routed(s["X"], s["W"], s["bias"], s["bank"], s["E"], s["I"], s["K"])
    assert np.array_equal(idx, i2)
    assert np.array_equal(bits(wt), bits(w2))
    p2, off2 = stable_gather(i2, s["N"])
    assert np.array_equal(perm, p2) and np.array_equal(off, off2)
    assert np.bincount(idx.ravel(), minlength=s["N"]).max() > 8     # some expert needs 2 passes
    assert drops == 0
    if prec == 0:
        for tk in range(s["T"]):
            assert max_err_rel_inf(out[tk], o2[tk]) <= TOL, tk
    else:
        assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16


@pytest.mark.parametrize("T,K,prec,E,I", [(1, 8, 0, 1024, 1536), (2, 8, 0, 1024, 1536),
                                         (1, 8, 1, 1024, 1536), (3, 5, 0, 1024, 1536),
                                         (2, 7, 1, 1024, 1536), (1, 1, 0, 1024, 1536),
                                         (2, 8, 0, 2048, 4096), (2, 8, 1, 2048, 4096),
                                         (1, 2, 1, 1024, 2048), (2, 1, 0, 1024, 2048),
                                         (1, 1, 0, 1024, 2048), (1, 1, 0, 2048, 2048),
                                         (1, 2, 1, 2048, 2048), (1, 4, 0, 2048, 2048)])
def test_moe_device_decode_path(gpu, orc, k3, T, K, prec, E, I):
    """At most 16 assignments (T * topk) take the decode kernels straight from the router's
    idx, without the gather: one tile per workgroup with K over up to 16 waves for few
    assignments, four tiles with K over two waves when they fill the chip (the 2048 x 4096
    cases); down and the combine in one kernel for one or two assignments (the 1-slot
    case), else down into per-slot rows and the combine kernel. With one tile per
    workgroup, K of at least four chunks and down + combine in one kernel (the 2048 x 2048
    cases), gate and up take workgroups of their own and down forms the activation from
    their fp32 sums; the run with the router's selection inside gate/up (no split) must
    give the same bits. Outputs
    against the oracle's per-slot sum (1e-4 * ||ref||inf with two-term
    activations, 2e-2 relative with one), row-major and tiled banks bit-identical, a
    NaN-scaled expert, and a dropped expert that contributes nothing and is counted."""
    N = 12
    say(f"case: device moe decode path T={T} K={K} prec={prec} E={E} I={I}")
    rng = np.random.default_rng(100 * T + K + prec)
    bank = [k3.gen_expert(E, I, 61, e) for e in range(N)]
    bank[5] = nan_scaled(k3, E, I, 61, 5)
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    _, idx0, _ = orc.moe_routed(X, W, None, bank, E, I, K)
    victim = int(idx0[0, 1]) if K > 1 else -1          # one slot: nothing dropped
    holed = list(bank)
    if victim >= 0:
        holed[victim] = None
    res = {}
    for layout in (gpu.K3D_LAYOUT_ROWS, gpu.K3D_LAYOUT_TILED):
        b = gpu.DevBank(holed, E, I, layout)
        try:
            res[layout] = gpu.moe_routed_device(b, X, W, None, K, prec=prec, inter=I)
            # no permutation asked for: the decode gate/up kernel selects the experts itself
            fused = gpu.moe_routed_device(b, X, W, None, K, prec=prec, inter=I, want_perm=False)
        finally:
            b.free()
        for i in (0, 1, 2, 5):                      # out, idx, wt, drops
            assert np.array_equal(np.asarray(fused[i]), np.asarray(res[layout][i])), (layout, i)
    r, t = res[gpu.K3D_LAYOUT_ROWS], res[gpu.K3D_LAYOUT_TILED]
    for a, b in zip(r, t):
        assert np.array_equal(np.asarray(a), np.asarray(b))
    out, idx, wt, perm, off, drops = r
    assert np.array_equal(idx, idx0)
    p2, off2 = stable_gather(idx0, N)
    assert np.array_equal(perm, p2) and np.array_equal(off, off2)
    assert drops == int((idx == victim).sum()) >= (1 if K > 1 else 0)
    for tk in range(T):
        acc = np.zeros(E, np.float32)
        for j in range(K):
            e = int(idx[tk, j])
            if e == victim:
                continue
            acc = acc + np.float32(wt[tk, j]) * orc.expert_ffn(X[tk], bank[e], E, I, act=1, wt=1.0)
        if prec == 0:
            assert max_err_rel_inf(out[tk], acc) <= TOL, tk
        else:
            assert np.linalg.norm(out[tk] - acc) / np.linalg.norm(acc) <= TOL_BF16, tk


def test_moe_device_tiled_decode_golden(gpu, wl, gold):
    """Full decode shape (7168 x 2048, 384 experts, top-8) from a tiled bank: the reference's
    golden routing and outputs for 8 tokens."""
    say("case: device moe tiled, decode shape, 8 tokens vs golden")
    W = wl.router_weights()
    X = wl.tokens(64)[:8]
    bank = gpu.DevBank(wl.lazy_bank(gold["router_idx"][:8]), wl.HIDDEN, wl.INTER,
                       gpu.K3D_LAYOUT_TILED)
    try:
        out, idx, wt, _, _, drops = gpu.moe_routed_device(bank, X, W, None, wl.TOPK, inter=wl.INTER)
    finally:
        bank.free()
    assert np.array_equal(idx, gold["router_idx"][:8])
    assert np.array_equal(bits(wt), bits(gold["router_wt"][:8]))
    assert drops == 0
    for t in range(8):
        assert max_err_rel_inf(out[t], gold["moe8_out"][t]) <= TOL, t


@pytest.mark.parametrize("T,hidden,N,K,biased", [
    (1, 7168, 384, 8, False), (1, 1001, 70, 5, True), (2, 1001, 70, 5, True),
    (3, 7168, 384, 8, True), (4, 8192, 96, 8, False), (2, 8200, 64, 4, True),
    (7, 7168, 384, 8, True), (31, 1001, 70, 5, True),
    (33, 1000, 70, 5, False), (64, 7168, 384, 8, False), (100, 520, 131, 16, True),
    (129, 7168, 384, 8, False), (300, 1000, 200, 5, True), (1100, 1000, 200, 5, True),
    (1024, 2304, 130, 8, False),
    (2, 1024, 1000, 8, True), (40, 512, 1500, 8, False), (20, 256, 2048, 16, True)])
def test_router_device_bit_exact(gpu, orc, T, hidden, N, K, biased):
    """Every partial kernel (a workgroup per expert for a few tokens up to 64 chunks of 128
    columns, one lane per chunk past that, the matrix cores for more tokens: fp64, and int8
    digit products from 1024 tokens when the rows are a multiple of 256 columns, else fp64
    again), widths that are not a multiple of the staging chunk (and an odd one: scalar
    loads), expert and token counts that are not multiples of the tiles: idx and weight
    bits equal to the oracle's per-token router."""
    say(f"case: router T={T} hidden={hidden} N={N} K={K} bias={biased}")
    rng = np.random.default_rng(T * 1000 + hidden)
    W = (rng.standard_normal((N, hidden)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32) if biased else None
    X = rng.standard_normal((T, hidden)).astype(np.float32)
    idx, wt = gpu.router_device(X, W, bias, K)
    say(f"  recomputed logits: {int(gpu.router_device.recomputed.sum())} over {T} tokens")
    assert gpu.router_device.recomputed.sum() <= max(2, T // 8)   # the fallback stays rare
    for t in range(T):
        i2, w2 = orc.router(X[t], W, bias, K)
        assert np.array_equal(idx[t], i2), t
        assert np.array_equal(bits(wt[t]), bits(w2)), t


def test_router_device_ties_and_nonfinite(gpu, orc):
    """Duplicate expert rows give equal choices (lowest index wins); a NaN and a -inf bias
    keep an expert from ever being chosen; fewer finite candidates than topk give idx 0,
    weight 0 (reference first-strict-max rule)."""
    say("case: router ties and non-finite choices")
    rng = np.random.default_rng(5)
    N, hidden, K = 12, 256, 6
    W = (rng.standard_normal((N, hidden)) * 0.05).astype(np.float32)
    W[7] = W[2]
    W[9] = W[2]
    X = rng.standard_normal((3, hidden)).astype(np.float32)
    bias = np.zeros(N, np.float32)
    bias[4] = np.nan
    bias[5] = -np.inf
    for b in (None, bias):
        idx, wt = gpu.router_device(X, W, b, K)
        for t in range(3):
            i2, w2 = orc.router(X[t], W, b, K)
            assert np.array_equal(idx[t], i2), (t, idx[t], i2)
            assert np.array_equal(bits(wt[t]), bits(w2)), t
    allbad = np.full(N, -np.inf, np.float32)
    allbad[:3] = 0.0
    idx, wt = gpu.router_device(X, W, allbad, K)
    for t in range(3):
        i2, w2 = orc.router(X[t], W, allbad, K)
        assert np.array_equal(idx[t], i2) and np.array_equal(bits(wt[t]), bits(w2))
        assert list(idx[t][3:]) == [0, 0, 0] and not wt[t][3:].any()


@pytest.mark.parametrize("T", [3, 9])
def test_router_device_ties_across_groups(gpu, orc, T):
    """384 experts, top-8: the selection runs in two levels (each wave the top 8 of its 64
    experts, then wave 0 over the candidates). Equal choices in different groups (experts
    2, 70 and 200 share a row, scaled up so that they are chosen) still go to the lowest
    index first; NaN and -inf biases in other groups are never chosen; with three finite
    candidates in three groups the rest are idx 0, weight 0. T = 3 scores in the small
    router, T = 9 in the matrix-core partials."""
    say(f"case: router ties across expert groups T={T}")
    rng = np.random.default_rng(11 + T)
    N, hidden, K = 384, 512, 8
    W = (rng.standard_normal((N, hidden)) * 0.02).astype(np.float32)
    W[2] = W[2] * 4.0
    W[70] = W[2]
    W[200] = W[2]
    X = rng.standard_normal((T, hidden)).astype(np.float32)
    X[:, :] = np.abs(X) * np.sign(W[2])[None, :]       # the shared row scores high
    bias = np.zeros(N, np.float32)
    bias[130] = np.nan
    bias[320] = -np.inf
    for b in (None, bias):
        idx, wt = gpu.router_device(X, W, b, K)
        for t in range(T):
            i2, w2 = orc.router(X[t], W, b, K)
            assert np.array_equal(idx[t], i2), (t, idx[t], i2)
            assert np.array_equal(bits(wt[t]), bits(w2)), t
            assert list(idx[t][:3]) == [2, 70, 200], idx[t]
    few = np.full(N, -np.inf, np.float32)
    few[[5, 150, 383]] = 0.0
    idx, wt = gpu.router_device(X, W, few, K)
    for t in range(T):
        i2, w2 = orc.router(X[t], W, few, K)
        assert np.array_equal(idx[t], i2) and np.array_equal(bits(wt[t]), bits(w2))
        assert list(idx[t][3:]) == [0] * 5 and not wt[t][3:].any()


@pytest.mark.parametrize("hidden", [1024, 7168])
@pytest.mark.parametrize("ntok", [2, 40, 200])
@pytest.mark.parametrize("scale", [1.0, -16.0])
def test_router_device_uncertified_logits(gpu, orc, hidden, ntok, scale):
    """Rows built so that a chunked fp64 sum and the reference's sequential chain round to
    different floats (1 + 2^-24 - 2^-52 then 2^-53 terms: the chain ties to even at every
    step, a chunked sum does not), times a power of two (the roundings scale with it).
    Expert 2's logit is exactly `scale`, a tie with the crafted experts under the reference
    (lowest index first), and the three are chosen first (a bias lifts them when the scale
    is negative), so both the order of idx and the weight bits would expose a wrong logit.
    At scale -16 the two candidate floats of a crafted logit have scores 30 ulps apart, so
    the router must run the reference's chain for them; at scale 1 the scores of the two
    candidates may coincide, which certifies the score without the chain."""
    say(f"case: router uncertified logits hidden={hidden} ntok={ntok} scale={scale}")
    N, K = 16, 4
    rng = np.random.default_rng(hidden)
    W = (rng.standard_normal((N, hidden)) * 1e-3).astype(np.float32)
    crafted = np.full(hidden, 2.0 ** -53, np.float32)
    crafted[:3] = [1.0, 2.0 ** -24, -2.0 ** -52]
    for e in (5, 11):
        W[e] = crafted * np.float32(scale)
    W[2] = 0.0
    W[2, 0] = scale
    bias = None
    if scale < 0:
        bias = np.zeros(N, np.float32)
        bias[[2, 5, 11]] = 1.0
    X = np.stack([np.ones(hidden, np.float32)] +
                 [rng.standard_normal(hidden).astype(np.float32) for _ in range(ntok - 1)])
    idx, wt = gpu.router_device(X, W, bias, K)
    rec = gpu.router_device.recomputed
    for t in range(ntok):
        i2, w2 = orc.router(X[t], W, bias, K)
        assert np.array_equal(idx[t], i2), (t, idx[t], i2)
        assert np.array_equal(bits(wt[t]), bits(w2)), t
    assert list(idx[0][:3]) == [2, 5, 11]
    if scale < 0:
        assert rec[0] >= 2      # both crafted logits went through the reference's chain


@pytest.mark.parametrize("ntok", [1, 2])
def test_moe_selection_in_gateup_uncertified(gpu, orc, k3, ntok):
    """The routed layer of a few tokens with no permutation asked for: the decode gate/up
    kernel selects the experts itself from the router's scored records. The crafted rows of
    test_router_device_uncertified_logits at scale -16 (two logits whose candidate floats'
    scores differ, so the reference's chain must run inside that kernel): idx and weight
    bits equal to the oracle's router, the output to the oracle's per-slot sum."""
    say(f"case: selection inside gate/up, uncertified logits, ntok={ntok}")
    E, I, N, K = 1024, 512, 16, 4
    rng = np.random.default_rng(77 + ntok)
    W = (rng.standard_normal((N, E)) * 1e-3).astype(np.float32)
    crafted = np.full(E, 2.0 ** -53, np.float32)
    crafted[:3] = [1.0, 2.0 ** -24, -2.0 ** -52]
    for e in (5, 11):
        W[e] = crafted * np.float32(-16.0)
    W[2] = 0.0
    W[2, 0] = -16.0
    bias = np.zeros(N, np.float32)
    bias[[2, 5, 11]] = 1.0
    X = np.stack([np.ones(E, np.float32)] +
                 [rng.standard_normal(E).astype(np.float32) for _ in range(ntok - 1)])
    bank = [k3.gen_expert(E, I, 91, e) for e in range(N)]
    b = gpu.DevBank(bank, E, I, gpu.K3D_LAYOUT_TILED)
    try:
        out, idx, wt, _, _, drops = gpu.moe_routed_device(b, X, W, bias, K, inter=I, want_perm=False)
    finally:
        b.free()
    assert drops == 0
    for t in range(ntok):
        i2, w2 = orc.router(X[t], W, bias, K)
        assert np.array_equal(idx[t], i2), (t, idx[t], i2)
        assert np.array_equal(bits(wt[t]), bits(w2)), t
        acc = np.zeros(E, np.float32)
        for j in range(K):
            acc = acc + np.float32(wt[t, j]) * orc.expert_ffn(X[t], bank[int(idx[t, j])], E, I, act=1, wt=1.0)
        assert max_err_rel_inf(out[t], acc) <= TOL, t
    assert list(idx[0][:3]) == [2, 5, 11]


def _graph_replay(gpu, bank_list, W, bias, E, I, N, K, T, prec, xs):
    """Capture the layer once in a HIP graph (k3d_graph_*), replay it with new input
    contents, with eager work and synchronisation between replays: every replay must equal
    the eager call on the same input, bit for bit."""
    import ctypes as C
    L = gpu.lib()
    bank = gpu.DevBank(bank_list, E, I, gpu.K3D_LAYOUT_TILED)
    dx = gpu.DevBuf(T * E * 4)
    dw = gpu.DevBuf(W.nbytes).upload(W)
    db = gpu.DevBuf(N * 4).upload(bias)
    out, idx, wt = gpu.DevBuf(T * E * 4), gpu.DevBuf(T * K * 4), gpu.DevBuf(T * K * 4)
    wsb = L.k3d_moe_ws(T, E, I, N, K, prec)
    ws = gpu.DevBuf(wsb)
    stream = L.k3d_stream_create()
    assert stream

    def call(st):
        gpu.check(L.k3d_moe_routed(out.ptr, idx.ptr, wt.ptr, dx.ptr, T, dw.ptr, db.ptr, bank.table.ptr,
                                   bank.layout, E, I, N, K, 1, 1.0, gpu.K3_ACT_SILU, 4.0, 25.0, prec,
                                   ws.ptr, wsb, None, None, None, st), "k3d_moe_routed")

    def results():
        return (out.download(np.empty((T, E), np.float32)), idx.download(np.empty((T, K), np.int32)),
                wt.download(np.empty((T, K), np.float32)))
    try:
        eager = []
        for x in xs:
            dx.upload(x)
            call(None)
            gpu.check(L.k3d_sync(None), "sync")
            eager.append(results())
        dx.upload(xs[0])
        gpu.check(L.k3d_graph_begin(stream), "graph_begin")
        call(stream)
        ex = C.c_void_p()
        gpu.check(L.k3d_graph_end(stream, C.byref(ex)), "graph_end")
        for rep in range(6):
            i = rep % len(xs)
            dx.upload(xs[i])
            call(None)                                   # eager work between replays
            gpu.check(L.k3d_sync(None), "sync")
            gpu.check(L.k3d_graph_launch(ex, stream), "graph_launch")
            gpu.check(L.k3d_sync(stream), "sync")
            got = results()
            for a, b in zip(got, eager[i]):
                assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                      b.view(np.uint32) if b.dtype == np.float32 else b), rep
        L.k3d_graph_destroy(ex)
    finally:
        L.k3d_stream_destroy(stream)
        for b in (dx, dw, db, out, idx, wt, ws):
            b.free()
        bank.free()


def test_moe_graph_replay_matches_eager(gpu, small_layer):
    """The decode-batch layer (8-token passes, two-term activations) captured in a HIP
    graph: every replay equals the eager call bit for bit."""
    s = small_layer
    say("case: graph replay vs eager")
    rng = np.random.default_rng(77)
    xs = [rng.standard_normal((s["T"], s["E"])).astype(np.float32) for _ in range(3)]
    _graph_replay(gpu, s["bank"], s["W"], s["bias"], s["E"], s["I"], s["N"], s["K"], s["T"], 0, xs)


@pytest.mark.parametrize("T,K", [(1, 8), (2, 8)])
def test_moe_graph_replay_decode_path(gpu, k3, T, K):
    """A few tokens captured in a HIP graph: the router's scored logits, the decode gate/up
    kernel that selects the experts itself, down and the combine. Every replay equals the
    eager call bit for bit."""
    E, I, N = 1024, 512, 16
    say(f"case: graph replay, decode path T={T} K={K}")
    rng = np.random.default_rng(90 + T)
    bank = [k3.gen_expert(E, I, 43, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32)
    xs = [rng.standard_normal((T, E)).astype(np.float32) for _ in range(3)]
    _graph_replay(gpu, bank, W, bias, E, I, N, K, T, 0, xs)


def test_moe_graph_replay_mixed_passes(gpu, k3):
    """The mixed pass lists (hot experts' 96-token passes on a side stream forked from the
    caller's and joined back) captured in a HIP graph: every replay equals the eager call
    bit for bit."""
    E, I, N, K, T = 1024, 512, 16, 4, 100
    say("case: graph replay vs eager, mixed pass lists")
    rng = np.random.default_rng(103)
    bank = [k3.gen_expert(E, I, 107, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    bias = np.zeros(N, np.float32)
    bias[[1, 9]] = 1.0
    xs = [rng.standard_normal((T, E)).astype(np.float32) for _ in range(3)]
    _graph_replay(gpu, bank, W, bias, E, I, N, K, T, 1, xs)

def test_moe_device_prefill_passes(gpu, orc, k3):
    """Prefill batches (>= 8 tokens per expert on average, bf16 activations) run 32-token
    passes with two MFMA column blocks: routing exact, outputs within 2e-2 relative of the
    oracle, row-major and tiled banks bit-identical, experts with more than 32 tokens."""
    E, I, N, K, T = 1024, 512, 8, 4, 97
    say(f"case: prefill passes E={E} I={I} N={N} K={K} T={T}")
    rng = np.random.default_rng(41)
    bank = [k3.gen_expert(E, I, 43, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    res = {}
    for layout in (gpu.K3D_LAYOUT_ROWS, gpu.K3D_LAYOUT_TILED):
        b = gpu.DevBank(bank, E, I, layout)
        try:
            res[layout] = gpu.moe_routed_device(b, X, W, None, K, prec=1, inter=I)
        finally:
            b.free()
    r, t = res[gpu.K3D_LAYOUT_ROWS], res[gpu.K3D_LAYOUT_TILED]
    for a, b in zip(r, t):
        assert np.array_equal(np.asarray(a), np.asarray(b))
    out, idx, wt, perm, off, drops = r
    o2, i2, w2 = orc.moe_routed(X, W, None, bank, E, I, K)
    assert np.array_equal(idx, i2)
    assert np.bincount(idx.ravel(), minlength=N).max() > 32       # several passes per expert
    assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16
    assert max_err_rel_inf(out, o2) <= 5e-2


def test_moe_device_prefill_96_passes(gpu, orc, k3):
    """Very large prefill batches on a tiled bank (>= 64 tokens per expert on average) run
    96-token passes with K staged 128 columns at a time: routing exact, outputs within
    2e-2 relative of the oracle and equal to the row-major bank's 32-token passes (the
    same K order per token), ragged last passes, experts with 2-3 passes."""
    E, I, N, K, T = 1536, 1024, 8, 4, 400
    say(f"case: prefill 96-token passes E={E} I={I} N={N} K={K} T={T}")
    rng = np.random.default_rng(59)
    bank = [k3.gen_expert(E, I, 67, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    res = {}
    for layout in (gpu.K3D_LAYOUT_ROWS, gpu.K3D_LAYOUT_TILED):
        b = gpu.DevBank(bank, E, I, layout)
        try:
            res[layout] = gpu.moe_routed_device(b, X, W, None, K, prec=1, inter=I)
        finally:
            b.free()
    out, idx, wt, perm, off, drops = res[gpu.K3D_LAYOUT_TILED]
    o2, i2, w2 = orc.moe_routed(X, W, None, bank, E, I, K)
    assert np.array_equal(idx, i2)
    cnt = np.bincount(idx.ravel(), minlength=N)
    assert cnt.max() > 192 and (cnt % 96 != 0).any()
    assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16
    assert max_err_rel_inf(out, o2) <= 5e-2
    rows_out = np.asarray(res[gpu.K3D_LAYOUT_ROWS][0])
    assert np.array_equal(np.asarray(res[gpu.K3D_LAYOUT_ROWS][1]), idx)
    assert np.abs(out - rows_out).max() <= 1e-6 * np.abs(rows_out).max()


@pytest.mark.parametrize("prec", [0, 1])
def test_moe_device_gather_many_workgroups(gpu, orc, k3, prec):
    """More than 2048 assignments take the gather over many workgroups (per-chunk counts,
    one scan, per-chunk stable placement; the last chunk ragged): perm and offsets equal to
    a stable argsort of idx, a missing expert's assignments counted as drops and left out
    of the output, experts without tokens, and outputs against the oracle's."""
    E, I, N, K, T = 512, 512, 64, 8, 700
    say(f"case: gather over many workgroups T={T} K={K} N={N} prec={prec}")
    rng = np.random.default_rng(83)
    bank = [k3.gen_expert(E, I, 89, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    W[[3, 40]] *= 0.0
    bias = np.zeros(N, np.float32)
    bias[[3, 40]] = -1e30                        # never chosen: experts without tokens
    X = rng.standard_normal((T, E)).astype(np.float32)
    _, idx0, _ = orc.moe_routed(X, W, bias, bank, E, I, K)
    victim = int(np.bincount(idx0.ravel(), minlength=N).argmax())
    holed = list(bank)
    holed[victim] = None
    b = gpu.DevBank(holed, E, I, gpu.K3D_LAYOUT_TILED)
    try:
        out, idx, wt, perm, off, drops = gpu.moe_routed_device(b, X, W, bias, K, prec=prec, inter=I)
    finally:
        b.free()
    assert np.array_equal(idx, idx0)
    cnt = np.bincount(idx.ravel(), minlength=N)
    assert idx.size > 2048 and cnt[3] == 0 and cnt[40] == 0
    p2, off2 = stable_gather(idx0, N)
    assert np.array_equal(perm, p2) and np.array_equal(off, off2)
    assert drops == int(cnt[victim]) > 0
    o2, _, _ = orc.moe_routed(X, W, bias, bank, E, I, K)
    for tk in np.nonzero((idx == victim).any(axis=1))[0]:     # the victim contributes nothing
        acc = np.zeros(E, np.float32)
        for j in range(K):
            e = int(idx[tk, j])
            if e != victim:
                acc = acc + np.float32(wt[tk, j]) * orc.expert_ffn(X[tk], bank[e], E, I, act=1, wt=1.0)
        o2[tk] = acc
    if prec == 0:
        for tk in range(T):
            assert max_err_rel_inf(out[tk], o2[tk]) <= TOL, tk
    else:
        assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16


@pytest.mark.parametrize("T,K,I", [(2, 8, 512), (24, 4, 512), (1, 2, 2048)])
def test_moe_experts_given_routing_invalid_slots(gpu, orc, k3, T, K, I):
    """k3d_moe_experts with a caller's routing: slots whose expert index lies outside the
    bank (-1, N, 1000) and slots of an absent expert contribute nothing; drops counts only
    the absent expert's slots; the rest equals the oracle's per-slot sum in slot order.
    (2, 8): 16 assignments, the decode kernels; (1, 2): down and the combine in one
    kernel; (24, 4): the gather path."""
    E, N = 1024, 12
    say(f"case: given routing with invalid slots T={T} K={K} I={I}")
    rng = np.random.default_rng(200 + T)
    bank = [k3.gen_expert(E, I, 211, e) for e in range(N)]
    holed = list(bank)
    holed[7] = None
    X = rng.standard_normal((T, E)).astype(np.float32)
    idx = rng.integers(0, N, size=(T, K)).astype(np.int32)
    if T > 1:
        idx[0, 1] = -1
        idx[1, 0] = N
        idx[-1, K - 1] = 1000
        idx[0, 0] = 7
    else:                       # one token: an absent slot beside a valid one
        idx[0] = [3, 7]
    wt = (rng.random((T, K)) + 0.1).astype(np.float32)
    b = gpu.DevBank(holed, E, I, gpu.K3D_LAYOUT_TILED)
    try:
        out, off, drops = gpu.moe_experts_device(b, X, idx, wt, N, prec=0, hidden=E, inter=I)
    finally:
        b.free()
    valid = (idx >= 0) & (idx < N)
    assert drops == int(((idx == 7) & valid).sum())
    assert off[N] == int(valid.sum())
    for tk in range(T):
        acc = np.zeros(E, np.float32)
        for j in range(K):
            e = int(idx[tk, j])
            if 0 <= e < N and holed[e] is not None:
                acc = acc + np.float32(wt[tk, j]) * orc.expert_ffn(X[tk], bank[e], E, I, act=1, wt=1.0)
        assert max_err_rel_inf(out[tk], acc) <= TOL, tk


def test_moe_experts_two_lists_invalid_slots(gpu, orc, k3):
    """k3d_moe_experts with a caller's routing in the two-list regime (bf16 activations,
    tiled bank, 8-32 assignments per expert on average): four hot experts in the 96-token
    list, cold ones in one 8-token pass each, one cold expert absent from the bank and
    slots outside the bank (-1, N, 1000). Drops count only the absent expert's slots, the
    offsets only valid slots, and every token's output is the oracle's per-slot sum
    without the dropped and invalid slots (2e-2 relative)."""
    E, I, N, K, T = 1024, 512, 12, 4, 40
    say(f"case: two pass lists with invalid slots E={E} I={I} N={N} K={K} T={T}")
    bank = [k3.gen_expert(E, I, 223, e) for e in range(N)]
    holed = list(bank)
    holed[7] = None
    rng = np.random.default_rng(227)
    X = rng.standard_normal((T, E)).astype(np.float32)
    t = np.arange(T)
    idx = np.stack([t % 4, (t + 1) % 4, 4 + t % 8,
                    np.where(t < 20, 4 + (t + 3) % 8, (t + 2) % 4)], axis=1).astype(np.int32)
    idx[0, 1] = -1
    idx[1, 0] = N
    idx[-1, K - 1] = 1000
    wt = (rng.random((T, K)) + 0.1).astype(np.float32)
    valid = (idx >= 0) & (idx < N)
    cnt = np.bincount(idx[valid], minlength=N)
    assert 8 * N <= T * K < 32 * N                                   # the two-list regime
    assert (cnt[:4] > 8).all() and (cnt[4:] <= 8).all() and cnt[7] > 0
    b = gpu.DevBank(holed, E, I, gpu.K3D_LAYOUT_TILED)
    try:
        out, off, drops = gpu.moe_experts_device(b, X, idx, wt, N, prec=1, hidden=E, inter=I)
    finally:
        b.free()
    assert drops == int(cnt[7])
    assert off[N] == int(valid.sum())
    o2 = np.zeros((T, E), np.float32)
    for tk in range(T):
        for j in range(K):
            e = int(idx[tk, j])
            if 0 <= e < N and holed[e] is not None:
                o2[tk] += np.float32(wt[tk, j]) * orc.expert_ffn(X[tk], bank[e], E, I, act=1, wt=1.0)
    assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16
    for tk in range(T):
        assert max_err_rel_inf(out[tk], o2[tk]) <= 5e-2, tk


def test_moe_device_mixed_passes(gpu, orc, k3):
    """Moderate batches on a tiled bank (8-32 tokens per expert on average) run one 8-token
    pass per expert of at most 8 assignments, and the experts holding more get the prefill
    kernel's 96-token passes from a second pass list: three biased experts take every token
    (100 each: two passes, the second ragged), the rest a few each (both lists hold some).
    Routing exact, outputs within 2e-2 relative of the oracle and equal to the row-major
    bank's (32-token passes throughout, the same K order per token)."""
    E, I, N, K, T = 1024, 512, 16, 4, 100
    say(f"case: mixed pass lists E={E} I={I} N={N} K={K} T={T}")
    rng = np.random.default_rng(97)
    bank = [k3.gen_expert(E, I, 101, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    bias = np.zeros(N, np.float32)
    bias[[0, 6, 13]] = 1.0
    X = rng.standard_normal((T, E)).astype(np.float32)
    res = {}
    for layout in (gpu.K3D_LAYOUT_ROWS, gpu.K3D_LAYOUT_TILED):
        b = gpu.DevBank(bank, E, I, layout)
        try:
            res[layout] = gpu.moe_routed_device(b, X, W, bias, K, prec=1, inter=I)
        finally:
            b.free()
    out, idx, wt, perm, off, drops = res[gpu.K3D_LAYOUT_TILED]
    o2, i2, w2 = orc.moe_routed(X, W, bias, bank, E, I, K)
    assert np.array_equal(idx, i2)
    cnt = np.bincount(idx.ravel(), minlength=N)
    rest = cnt[[e for e in range(N) if e not in (0, 6, 13)]]
    assert (cnt[[0, 6, 13]] == T).all() and rest.max() <= 32
    assert (rest <= 8).any() and (rest > 8).any()                   # both lists hold experts
    p2, off2 = stable_gather(i2, N)
    assert np.array_equal(perm, p2) and np.array_equal(off, off2)
    assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16
    rows_out = np.asarray(res[gpu.K3D_LAYOUT_ROWS][0])
    assert np.abs(out - rows_out).max() <= 1e-6 * np.abs(rows_out).max()


def test_moe_device_prefill_48_passes(gpu, orc, k3):
    """Large prefill batches on a tiled bank (>= 32 tokens per expert on average) run
    48-token passes with K staged 256 columns at a time: routing exact, outputs within 2e-2
    relative of the oracle, and equal to the row-major bank's 32-token passes, which take
    the same K order per token (ragged last passes, experts with 2-4 passes)."""
    E, I, N, K, T = 1536, 1024, 8, 4, 200
    say(f"case: prefill 48-token passes E={E} I={I} N={N} K={K} T={T}")
    rng = np.random.default_rng(47)
    bank = [k3.gen_expert(E, I, 53, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    res = {}
    for layout in (gpu.K3D_LAYOUT_ROWS, gpu.K3D_LAYOUT_TILED):
        b = gpu.DevBank(bank, E, I, layout)
        try:
            res[layout] = gpu.moe_routed_device(b, X, W, None, K, prec=1, inter=I)
        finally:
            b.free()
    out, idx, wt, perm, off, drops = res[gpu.K3D_LAYOUT_TILED]
    o2, i2, w2 = orc.moe_routed(X, W, None, bank, E, I, K)
    assert np.array_equal(idx, i2)
    cnt = np.bincount(idx.ravel(), minlength=N)
    assert cnt.max() > 96 and (cnt % 48 != 0).any()
    assert np.linalg.norm(out - o2) / np.linalg.norm(o2) <= TOL_BF16
    assert max_err_rel_inf(out, o2) <= 5e-2
    rows_out = np.asarray(res[gpu.K3D_LAYOUT_ROWS][0])
    assert np.array_equal(np.asarray(res[gpu.K3D_LAYOUT_ROWS][1]), idx)
    assert np.abs(out - rows_out).max() <= 1e-6 * np.abs(rows_out).max()


def shared_ref(orc, X, w1, w3, w2, hidden, inter):
    """The reference's shared tail per token: bf16 GEMVs (fp64 accumulation) and SiLU-GLU."""
    out = np.empty((X.shape[0], hidden), np.float32)
    for t in range(X.shape[0]):
        g = orc.matmul_bf16(X[t], w1.reshape(inter, hidden))
        u = orc.matmul_bf16(X[t], w3.reshape(inter, hidden))
        a = orc.silu_glu(np.concatenate([g, u]), inter)
        out[t] = orc.matmul_bf16(a, w2.reshape(hidden, inter))
    return out


@pytest.mark.parametrize("T,prec", [(5, 0), (40, 0), (70, 1), (300, 1)])
def test_shared_expert_vs_oracle(gpu, orc, k3, T, prec):
    """The bf16 dense shared expert on the matrix cores against the reference's bf16 GEMV
    composition: 1e-4 * ||ref||inf with two-term activations, 2e-2 relative with one (32-
    token passes, the last one ragged); the accumulate form adds onto the routed output with
    one fp32 add."""
    hidden, inter = 1024, 512
    say(f"case: shared expert T={T} prec={prec}")
    w1 = k3.gen_bf16_normal(inter * hidden, 101, 0.0, 0.02)
    w3 = k3.gen_bf16_normal(inter * hidden, 102, 0.0, 0.02)
    w2 = k3.gen_bf16_normal(hidden * inter, 103, 0.0, 0.02)
    X = k3.gen_normal(T * hidden, 104).reshape(T, hidden)
    ref = shared_ref(orc, X, w1, w3, w2, hidden, inter)
    got = gpu.shared_expert_device(X, w1, w3, w2, hidden, inter, prec=prec)
    if prec == 0:
        assert max_err_rel_inf(got, ref) <= TOL
    else:
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= TOL_BF16
    y0 = k3.gen_normal(T * hidden, 105).reshape(T, hidden)
    got2 = gpu.shared_expert_device(X, w1, w3, w2, hidden, inter, prec=prec, y0=y0)
    assert np.array_equal(got2, (y0 + got).astype(np.float32))
