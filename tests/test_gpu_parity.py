# SPDX-License-Identifier: Apache-2.0
"""GPU parity through the C ABI (libk3amd.so) against the oracle and the reference's
golden data. Tolerances: max|err| <= 1e-4 * ||ref||inf for the fp32-accurate paths,
2e-2 relative for the bf16-activation (prefill) precision; indices and permutations
bit-exact; MXFP4 dequantisation exact."""
import sys

import numpy as np
import pytest

import make_golden
from conftest import max_err_rel_inf

pytestmark = pytest.mark.gpu
TOL = 1e-4          # fp32-accumulated GEMV paths
TOL_BF16 = 2e-2     # bf16-activation (prefill) path


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_dequant_exact_on_checkpoint_bytes(gpu, fx):
    say("case: dequant mxfp4.json")
    rows, pcols = fx["mx_packed"].shape
    got = gpu.mxfp4_dequant(fx["mx_packed"], fx["mx_scales"], rows, pcols, 32)
    assert np.array_equal(bits(got), bits(fx["mx_expected"]))


def test_gemv_decode_shape(gpu, wl, gold):
    say("case: gemv 2048x7168")
    packed, scales, x = wl.gemv_inputs()
    y = gpu.matmul_mxfp4(x, packed, scales, wl.HIDDEN, 2048)
    assert max_err_rel_inf(y, gold["gemv_y"]) <= TOL


def test_gemv_bench_inputs(gpu, orc):
    say("case: gemv bench 3072x3584")
    inn, rows = 3584, 3072
    pk = orc.fill_b(rows * inn // 2, 777)
    sc = np.full(rows * inn // 32, 127, np.uint8)
    x = orc.fill_f(inn, 4242)
    want = orc.matmul_mxfp4(x, pk, sc, inn, rows)
    assert orc.fnv1a(want) == 0xA231061237B5579D
    assert max_err_rel_inf(gpu.matmul_mxfp4(x, pk, sc, inn, rows), want) <= TOL


@pytest.mark.parametrize("case", [c[0] for c in make_golden.edge_cases()])
def test_gemv_edge_cases(gpu, gold, case):
    say(f"case: gemv edge {case}")
    c = {c[0]: c for c in make_golden.edge_cases()}[case]
    _, pk, sc, x, inn, rows, group = c
    y = gpu.matmul_mxfp4(x, pk, sc, inn, rows, group)
    assert max_err_rel_inf(y, gold["edge_" + case]) <= TOL


@pytest.mark.parametrize("ntok,prec", [(1, 0), (2, 0), (3, 0), (1, 1), (2, 1)])
@pytest.mark.parametrize("rows,inn", [(2048, 7168), (37, 224), (100, 16384)])
def test_gemv_device_tokens(gpu, orc, ntok, prec, rows, inn):
    """k3d_matmul_mxfp4 on device buffers: one or two tokens take the kernel that splits
    fp32 activations itself (where they fit in LDS), three the split pass; every token
    against the oracle: 1e-4 * ||ref||inf with two-term activations, 2e-2 relative with
    one. Rows not a multiple of 16 and K not a multiple of 128 included."""
    say(f"case: device gemv rows={rows} in={inn} ntok={ntok} prec={prec}")
    rng = np.random.default_rng(rows + inn + 10 * ntok + prec)
    pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
    sc = rng.integers(118, 128, rows * inn // 32, dtype=np.uint8)
    sc[rng.integers(0, sc.size, 8)] = 255                  # NaN bytes: blocks of zeros
    X = rng.standard_normal((ntok, inn)).astype(np.float32)
    L = gpu.lib()
    dp, ds = gpu.DevBuf(pk.nbytes).upload(pk), gpu.DevBuf(sc.nbytes).upload(sc)
    dx, dy = gpu.DevBuf(X.nbytes).upload(X), gpu.DevBuf(ntok * rows * 4)
    ws = gpu.DevBuf(max(L.k3d_matmul_mxfp4_ws(ntok, inn), 16))
    try:
        gpu.check(L.k3d_matmul_mxfp4(dy.ptr, dx.ptr, ntok, dp.ptr, ds.ptr, inn, rows, prec,
                                     ws.ptr, ws.nbytes, None), "k3d_matmul_mxfp4")
        Y = dy.download(np.empty((ntok, rows), np.float32))
    finally:
        for b in (dp, ds, dx, dy, ws):
            b.free()
    for t in range(ntok):
        want = orc.matmul_mxfp4(X[t], pk, sc, inn, rows)
        if prec == 0:
            assert max_err_rel_inf(Y[t], want) <= TOL
        else:
            assert np.linalg.norm(Y[t] - want) / np.linalg.norm(want) <= TOL_BF16


@pytest.mark.parametrize("ntok,prec", [(1, 0), (2, 0), (1, 1), (2, 1)])
def test_gemv_eight_row_tiles_bit_identical(gpu, orc, ntok, prec):
    """A matrix with fewer 16-row tiles than the chip has CUs (2048 x 7168) runs 8-row tiles
    with two 512-column chunks per wave; 4096 rows run 16-row tiles. Rows are independent,
    so the first 2048 rows alone give the 4096-row matrix's first 2048 outputs bit for bit;
    both against the oracle too."""
    say(f"case: gemv 8-row vs 16-row tiles ntok={ntok} prec={prec}")
    inn, big, small = 7168, 4096, 2048
    rng = np.random.default_rng(77 + ntok + 10 * prec)
    pk = rng.integers(0, 256, big * inn // 2, dtype=np.uint8)
    sc = rng.integers(118, 128, big * inn // 32, dtype=np.uint8)
    sc[rng.integers(0, sc.size, 16)] = 255
    X = rng.standard_normal((ntok, inn)).astype(np.float32)
    L = gpu.lib()

    def run(rows):
        p, s = pk[:rows * inn // 2], sc[:rows * inn // 32]
        dp, ds = gpu.DevBuf(p.nbytes).upload(p), gpu.DevBuf(s.nbytes).upload(s)
        dx, dy = gpu.DevBuf(X.nbytes).upload(X), gpu.DevBuf(ntok * rows * 4)
        ws = gpu.DevBuf(max(L.k3d_matmul_mxfp4_ws(ntok, inn), 16))
        try:
            gpu.check(L.k3d_matmul_mxfp4(dy.ptr, dx.ptr, ntok, dp.ptr, ds.ptr, inn, rows, prec,
                                         ws.ptr, ws.nbytes, None), "k3d_matmul_mxfp4")
            return dy.download(np.empty((ntok, rows), np.float32))
        finally:
            for b in (dp, ds, dx, dy, ws):
                b.free()

    Yb, Ys = run(big), run(small)
    assert np.array_equal(bits(Ys), bits(Yb[:, :small]))
    want = orc.matmul_mxfp4(X[0], pk[:small * inn // 2], sc[:small * inn // 32], inn, small)
    if prec == 0:
        assert max_err_rel_inf(Ys[0], want) <= TOL
    else:
        assert np.linalg.norm(Ys[0] - want) / np.linalg.norm(want) <= TOL_BF16


def test_dense_gemv_f32_bf16_identical(gpu, orc):
    """k3_matmul_bf16 equals k3_matmul on the widened weights bit for bit, over arbitrary
    finite bf16 patterns (the reference's own check, test_ops.c:811-848)."""
    say("case: bf16 vs f32 gemv identity")
    rng = np.random.default_rng(11)
    for inn, out in ((257, 129), (7168, 300)):
        Wb = (rng.integers(0, 65536, (out, inn)).astype(np.uint16) & 0x7F7F)
        Wf = (Wb.astype(np.uint32) << 16).view(np.float32)
        x = rng.standard_normal(inn).astype(np.float32)
        assert np.array_equal(bits(gpu.matmul(x, Wf)), bits(gpu.matmul_bf16(x, Wb)))


@pytest.mark.parametrize("shape", [(257, 129), (7168, 2048), (2048, 7168)])
def test_dense_gemv_bf16_vs_oracle(gpu, orc, k3, shape):
    say(f"case: bf16 gemv {shape}")
    inn, out = shape
    Wb = k3.gen_bf16_normal(inn * out, 31, 0.0, 0.02).reshape(out, inn)
    x = k3.gen_normal(inn, 32)
    assert max_err_rel_inf(gpu.matmul_bf16(x, Wb), orc.matmul_bf16(x, Wb)) <= TOL
    Wf = (Wb.astype(np.uint32) << 16).view(np.float32)
    assert max_err_rel_inf(gpu.matmul(x, Wf), orc.matmul(x, Wf)) <= TOL


def test_router_fixture(gpu, fx):
    say("case: router.json")
    W, bias, X = fx["rt_W"], fx["rt_bias"], fx["rt_x"]
    K = int(fx["rt_topk"])
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    for r in range(X.shape[0]):
        idx, w = gpu.router(X[r], W, bias, K)
        assert set(idx.tolist()) == set(fx["rt_idx"][r].tolist())
        for a in range(K):
            b = list(fx["rt_idx"][r]).index(idx[a])
            assert abs(w[a] - fx["rt_wt"][r][b]) <= atol + rtol * abs(fx["rt_wt"][r][b])


def test_router_decode_bit_exact(gpu, wl, gold):
    say("case: router 384x7168 top-8, 64 tokens")
    W = wl.router_weights()
    X = wl.tokens(64)
    for t in range(64):
        idx, w = gpu.router(X[t], W, None, wl.TOPK)
        assert np.array_equal(idx, gold["router_idx"][t]), t
        assert np.array_equal(bits(w), bits(gold["router_wt"][t])), t


def test_situ_and_rmsnorm_fixtures(gpu, fx):
    say("case: situ_glu.json, rmsnorm.json")
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    X, Y = fx["situ_in"], fx["situ_out"]
    n = Y.shape[1]
    for r in range(X.shape[0]):
        y = gpu.situ_glu(X[r], n, float(fx["situ_b1"]), float(fx["situ_b2"]))
        assert np.all(np.abs(y - Y[r]) <= atol + rtol * np.abs(Y[r]))
    X, Y, w = fx["rms_in"], fx["rms_out"], fx["rms_w"]
    for r in range(X.shape[0]):
        y = gpu.rmsnorm(X[r], w, float(fx["rms_eps"]))
        assert np.all(np.abs(y - Y[r]) <= atol + rtol * np.abs(Y[r]))


@pytest.mark.parametrize("act", [1, 0])
def test_expert_ffn_decode(gpu, wl, gold, act):
    say(f"case: expert ffn act={act}")
    e0, xe = wl.expert(0), wl.expert_input()
    out = gpu.expert_ffn(xe, e0, wl.HIDDEN, wl.INTER, act=act, wt=0.125)
    assert max_err_rel_inf(out, gold["expert_silu" if act == 1 else "expert_situ"]) <= TOL


@pytest.mark.parametrize("act", [1, 0])
def test_expert_ffn_decode_tiled_timed_path(gpu, wl, gold, act):
    """The call the benchmark times for one expert's FFN: k3d_moe_experts with one
    assignment (combine weight 0.125) on a tiled 7168 -> 2048 bank (gate and up in
    workgroups of their own, then down + combine in one kernel), against the compiled
    reference's golden, with the expert placed at entry 3 of a 6-entry table."""
    import ctypes as C
    say(f"case: expert ffn, tiled timed path, act={act}")
    L = gpu.lib()
    E, I, N = wl.HIDDEN, wl.INTER, 6
    bank = gpu.DevBank([None, None, None, wl.expert(0), None, None], E, I, gpu.K3D_LAYOUT_TILED)
    x = gpu.DevBuf(E * 4).upload(wl.expert_input())
    out = gpu.DevBuf(E * 4)
    idx = gpu.DevBuf(4).upload(np.array([3], np.int32))
    wt = gpu.DevBuf(4).upload(np.array([0.125], np.float32))
    drops = gpu.DevBuf(4)
    ws = gpu.DevBuf(L.k3d_moe_ws(1, E, I, N, 1, 0))
    try:
        out.upload(np.full(E, np.nan, np.float32))
        gpu.check(L.k3d_moe_experts(out.ptr, idx.ptr, wt.ptr, x.ptr, 1, bank.table.ptr,
                                    gpu.K3D_LAYOUT_TILED, E, I, N, 1, act, 4.0, 25.0, 0, ws.ptr,
                                    ws.nbytes, None, None, drops.ptr, None), "k3d_moe_experts")
        gpu.check(L.k3d_sync(None))
        got = out.download(np.empty(E, np.float32))
        nd = int(drops.download(np.empty(1, np.int32))[0])
    finally:
        for b in (x, out, idx, wt, drops, ws):
            b.free()
        bank.free()
    assert nd == 0
    assert max_err_rel_inf(got, gold["expert_silu" if act == 1 else "expert_situ"]) <= TOL


def test_moe_routed_8_tokens_golden(gpu, wl, gold):
    say("case: moe routed T=8 vs golden")
    W = wl.router_weights()
    X = wl.tokens(64)[:8]
    bank = wl.lazy_bank(gold["router_idx"][:8])
    out, idx, wt = gpu.moe_routed(X, W, None, bank, wl.HIDDEN, wl.INTER, wl.TOPK)
    assert np.array_equal(idx, gold["router_idx"][:8])
    assert np.array_equal(bits(wt), bits(gold["router_wt"][:8]))
    for t in range(8):
        assert max_err_rel_inf(out[t], gold["moe8_out"][t]) <= TOL, t


def test_moe_routed_small_shapes_vs_oracle(gpu, orc, k3):
    """Ragged routing on a small layer: 24 experts, top-3, 37 tokens, hidden 256, inter 96,
    with a selection bias; every token's output, idx and weights."""
    say("case: moe routed small shapes")
    rng = np.random.default_rng(21)
    E, I, N, K, T = 256, 96, 24, 3, 37
    bank = [k3.gen_expert(E, I, 99, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    out, idx, wt = gpu.moe_routed(X, W, bias, bank, E, I, K)
    o2, i2, w2 = orc.moe_routed(X, W, bias, bank, E, I, K)
    assert np.array_equal(idx, i2)
    assert np.array_equal(bits(wt), bits(w2))
    for t in range(T):
        assert max_err_rel_inf(out[t], o2[t]) <= TOL, t


def test_moe_routed_prefill_precision(gpu, orc, k3):
    say("case: moe routed bf16 activations")
    rng = np.random.default_rng(22)
    E, I, N, K, T = 512, 256, 16, 4, 70
    bank = [k3.gen_expert(E, I, 7, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    out, idx, wt = gpu.moe_routed(X, W, None, bank, E, I, K, prec=1)
    o2, i2, _ = orc.moe_routed(X, W, None, bank, E, I, K)
    assert np.array_equal(idx, i2)
    rel = np.linalg.norm(out - o2) / np.linalg.norm(o2)
    assert rel <= TOL_BF16


def test_moe_dropped_expert(gpu, orc, k3):
    """A missing expert contributes nothing and is counted (k3_ops.c:616-626)."""
    say("case: moe dropped expert")
    rng = np.random.default_rng(23)
    E, I, N, K, T = 256, 64, 8, 2, 12
    bank = [k3.gen_expert(E, I, 3, e) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    _, idx, _ = orc.moe_routed(X, W, None, bank, E, I, K)
    victim = int(idx[0, 0])
    holed = list(bank)
    holed[victim] = None
    before = k3.expert_drops()
    out, idx_g, wt = gpu.moe_routed(X, W, None, holed, E, I, K)
    assert k3.expert_drops() - before == int((idx_g == victim).sum())
    # expected: the oracle's per-slot sum without the victim's slots
    for t in range(T):
        acc = np.zeros(E, np.float32)
        for j in range(K):
            e = int(idx_g[t, j])
            if e == victim:
                continue
            acc = acc + np.float32(wt[t, j]) * orc.expert_ffn(X[t], bank[e], E, I, act=1, wt=1.0)
        assert max_err_rel_inf(out[t], acc) <= TOL


def test_moe_latent_fixture(gpu, fx):
    """ops/moe.json through k3_moe (resident fp32 experts) at the manifest tolerance."""
    say("case: k3_moe moe.json")
    import ctypes as C
    from test_oracle import moe_fixture
    cfg, W, x, y = moe_fixture(fx)
    c = gpu.K3Cfg()
    c.hidden, c.latent, c.moe_inter = int(cfg["hidden"]), int(cfg["latent"]), int(cfg["inter"])
    c.n_experts, c.topk, c.n_shared = int(cfg["n_experts"]), int(cfg["topk"]), int(cfg["n_shared"])
    c.moe_renorm, c.latent_norm = int(cfg["renorm"]), int(cfg["latent_norm"])
    c.routed_scale, c.rms_eps = float(cfg["routed_scale"]), float(cfg["rms_eps"])
    c.situ_b1, c.situ_b2 = float(cfg["b1"]), float(cfg["b2"])
    keep = {k: np.ascontiguousarray(v, np.float32) for k, v in W.items()}
    w = gpu.K3MoeW()
    for k in ("gate", "bias", "w1", "w3", "w2", "latent_norm", "down", "up", "sh1", "sh3", "sh2"):
        setattr(w, k, keep[k].ctypes.data)
    x = np.ascontiguousarray(x, np.float32).reshape(-1, c.hidden)
    T = x.shape[0]
    out = np.empty_like(x)
    idx = np.empty(c.topk, np.int32)
    wt = np.empty(c.topk, np.float32)
    scratch = np.empty(gpu.lib().k3_moe_scratch(C.byref(c)), np.float32)
    gpu.lib().k3_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(c), T, idx.ctypes.data,
                     wt.ctypes.data, scratch.ctypes.data)
    y = y.reshape(out.shape)
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    assert np.all(np.abs(out - y) <= atol + rtol * np.abs(y))
