# SPDX-License-Identifier: Apache-2.0
"""The oracle (oracle/k3_oracle.c) pinned before it is trusted:

  * the reference's own golden data: bench_kernels.c output hashes, mxfp4.json (real
    checkpoint bytes, exact, plus its swapped-nibble negative), router.json, situ_glu.json,
    rmsnorm.json, moe.json at the manifest tolerance;
  * the compiled reference (oracle/_ref) on this project's workloads, bit for bit;
  * what the mathematics fixes: exact rational evaluation of small GEMVs, closed-form
    dequantisation, tie-breaking by brute force, gather stability, NaN/short cases.
"""
from fractions import Fraction

import numpy as np
import pytest

import make_golden

# FNV-1a of the reference benchmark's outputs (benchmarks/bench_kernels.c:102-160), the
# same value in its AVX2 and scalar builds.
FNV_MXFP4_BENCH = 0xA231061237B5579D
FNV_BF16_BENCH = 0x83C8504A4CB3FAC6

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_bench_hashes_mxfp4(orc):
    inn, rows = 3584, 3072
    pk = orc.fill_b(rows * inn // 2, 777)
    sc = np.full(rows * inn // 32, 127, np.uint8)
    x = orc.fill_f(inn, 4242)
    assert orc.fnv1a(orc.matmul_mxfp4(x, pk, sc, inn, rows)) == FNV_MXFP4_BENCH


def test_bench_hashes_bf16(orc):
    W = orc.fill_bf16(12288 * 7168, 12345).reshape(12288, 7168)
    x = orc.fill_f(7168, 999)
    assert orc.fnv1a(orc.matmul_bf16(x, W)) == FNV_BF16_BENCH


def test_dequant_exact_on_checkpoint_bytes(orc, fx):
    rows, pcols = fx["mx_packed"].shape
    got = orc.mxfp4_dequant(fx["mx_packed"], fx["mx_scales"], rows, pcols, int(fx["mx_group"]))
    assert np.array_equal(bits(got), bits(fx["mx_expected"]))


def test_dequant_swapped_nibbles_is_detected(orc, fx):
    """Planting the classic mistake (low nibble = ODD element) in the oracle's input order
    reproduces the fixture's recorded wrong answer, and that answer differs from truth."""
    pk = fx["mx_packed"].copy()
    swapped = ((pk >> 4) | (pk << 4)).astype(np.uint8)
    rows, pcols = pk.shape
    got = orc.mxfp4_dequant(swapped, fx["mx_scales"], rows, pcols, 32)
    assert np.array_equal(got.ravel()[:64], fx["mx_swapped_first64"])
    assert not np.array_equal(got, fx["mx_expected"])


def test_dequant_closed_form(orc):
    rng = np.random.default_rng(1)
    rows, inn = 9, 96
    pk = rng.integers(0, 256, (rows, inn // 2), dtype=np.uint8)
    sc = rng.integers(0, 256, (rows, inn // 32), dtype=np.uint8)
    want = np.zeros((rows, inn), np.float32)
    for r in range(rows):
        for i in range(inn):
            b = int(pk[r, i // 2])
            code = (b >> 4) if i & 1 else (b & 15)
            s = int(sc[r, i // 32])
            want[r, i] = 0.0 if s == 255 else np.float32(E2M1[code]) * np.float32(2.0 ** (s - 127))
    got = orc.mxfp4_dequant(pk, sc, rows, inn // 2, 32)
    assert np.array_equal(bits(got), bits(want))


def test_gemv_against_exact_rationals(orc):
    """Every product is exact in double; the only rounding is the additions. Against the
    exact rational sum the fp32 result must be within one fp32 ulp plus double slack."""
    rng = np.random.default_rng(2)
    rows, inn = 6, 160
    pk = rng.integers(0, 256, (rows, inn // 2), dtype=np.uint8)
    sc = rng.integers(110, 140, (rows, inn // 32), dtype=np.uint8)
    x = rng.standard_normal(inn).astype(np.float32)
    y = orc.matmul_mxfp4(x, pk, sc, inn, rows)
    for r in range(rows):
        s = Fraction(0)
        for i in range(inn):
            b = int(pk[r, i // 2])
            code = (b >> 4) if i & 1 else (b & 15)
            s += Fraction(E2M1[code]) * Fraction(2) ** (int(sc[r, i // 32]) - 127) * Fraction(float(x[i]))
        exact = float(s)
        assert abs(float(y[r]) - exact) <= abs(exact) * 2 ** -23 + 1e-30


def test_gemv_matches_dequant_then_matmul(orc):
    """test_expert.c:204-229 of the reference: fused MXFP4 GEMV vs dequantise + k3_matmul
    within 1e-6 relative."""
    rng = np.random.default_rng(3)
    rows, inn = 64, 3584
    pk = rng.integers(0, 256, (rows, inn // 2), dtype=np.uint8)
    sc = rng.integers(119, 128, (rows, inn // 32), dtype=np.uint8)
    x = rng.standard_normal(inn).astype(np.float32)
    a = orc.matmul_mxfp4(x, pk, sc, inn, rows)
    b = orc.matmul(x, orc.mxfp4_dequant(pk, sc, rows, inn // 2, 32))
    assert np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-30)) < 1e-6


def test_preconditions_abort():
    """Odd `in` and group > 64 abort (k3_ops.c:1383-1401); checked in a child process."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, 'oracle'); import numpy as np; from oracle import Oracle;"
            "o = Oracle(); o.matmul_mxfp4(np.zeros(3, np.float32), np.zeros(8, np.uint8),"
            " np.zeros(8, np.uint8), {inn}, 1, {g})")
    root = make_golden.ROOT
    for inn, g in ((3, 32), (64, 96)):
        r = subprocess.run([sys.executable, "-c", code.format(inn=inn, g=g)], cwd=root,
                           capture_output=True, text=True)
        assert r.returncode != 0 and "FATAL" in r.stderr


def test_router_fixture(orc, fx):
    """ops/router.json: index sets, and weights matched by id, at the manifest tolerance."""
    W, bias, X = fx["rt_W"], fx["rt_bias"], fx["rt_x"]
    K = int(fx["rt_topk"])
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    for r in range(X.shape[0]):
        idx, w = orc.router(X[r], W, bias, K)
        assert set(idx.tolist()) == set(fx["rt_idx"][r].tolist())
        for a in range(K):
            b = list(fx["rt_idx"][r]).index(idx[a])
            assert abs(w[a] - fx["rt_wt"][r][b]) <= atol + rtol * abs(fx["rt_wt"][r][b])


def test_router_bias_steers_selection_only(orc, fx):
    """Weights come from the unbiased scores: removing the bias on the fixture changes the
    selection on the recorded number of rows."""
    W, bias, X = fx["rt_W"], fx["rt_bias"], fx["rt_x"]
    K = int(fx["rt_topk"])
    changed = sum(set(orc.router(X[r], W, bias, K)[0]) != set(orc.router(X[r], W, None, K)[0])
                  for r in range(X.shape[0]))
    assert changed == int(fx["rt_changed"])


def test_router_ties_go_to_lowest_index(orc):
    """Equal rows give bit-equal scores; the first strict maximum over ascending e wins,
    and idx comes out in descending score order."""
    rng = np.random.default_rng(4)
    W = rng.standard_normal((12, 64)).astype(np.float32) * 0.1
    W[7] = W[3]
    W[10] = W[3]
    x = rng.standard_normal(64).astype(np.float32)
    idx, w = orc.router(x, W, None, 12, renorm=0)
    order = [int(i) for i in idx]
    assert order.index(3) < order.index(7) < order.index(10)
    assert all(w[i] >= w[i + 1] for i in range(11))
    # brute force: stable sort by descending score gives the same order
    s = 1.0 / (1.0 + np.exp(-(W.astype(np.float64) @ x.astype(np.float64))))
    assert order[0] == int(np.argmax(s))


def test_router_no_candidate_and_renorm(orc):
    W = np.full((4, 8), np.nan, np.float32)
    idx, w = orc.router(np.ones(8, np.float32), W, None, 3)
    assert idx.tolist() == [0, 0, 0] and w.tolist() == [0.0, 0.0, 0.0]
    W = np.eye(4, 8, dtype=np.float32)
    idx, w = orc.router(np.arange(8, dtype=np.float32), W, None, 2, renorm=1, routed_scale=2.5)
    assert idx.tolist() == [3, 2]
    assert abs(float(w.sum()) - 2.5) < 1e-6


def test_situ_fixture_and_bound(orc, fx):
    X, Y = fx["situ_in"], fx["situ_out"]
    b1, b2 = float(fx["situ_b1"]), float(fx["situ_b2"])
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    n = Y.shape[1]
    for r in range(X.shape[0]):
        y = orc.situ_glu(X[r], n, b1, b2)
        assert np.all(np.abs(y - Y[r]) <= atol + rtol * np.abs(Y[r]))
        assert np.abs(y).max() <= b1 * b2 + 1e-2


def test_silu_closed_form(orc):
    x = np.linspace(-30, 30, 200, dtype=np.float32)
    gu = np.concatenate([x, np.full_like(x, 1.5)])
    y = orc.silu_glu(gu, x.size)
    want = (x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))) * 1.5
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))


def test_rmsnorm_fixture(orc, fx):
    X, Y, w = fx["rms_in"], fx["rms_out"], fx["rms_w"]
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    for r in range(X.shape[0]):
        y = orc.rmsnorm(X[r], w, float(fx["rms_eps"]))
        assert np.all(np.abs(y - Y[r]) <= atol + rtol * np.abs(Y[r]))


def moe_fixture(fx):
    cfg = dict(hidden=fx["moe_hidden"], latent=fx["moe_latent"], inter=fx["moe_moe_inter"],
               n_experts=fx["moe_n_experts"], topk=fx["moe_top_k"], n_shared=fx["moe_n_shared"],
               renorm=fx["moe_renorm"], latent_norm=fx["moe_latent_norm"],
               routed_scale=fx["moe_routed_scale"], rms_eps=fx["moe_rms_eps"],
               b1=fx["moe_situ_b1"], b2=fx["moe_situ_b2"])
    n = int(cfg["n_experts"])
    W = dict(gate=fx["moe_t_gate_weight"], bias=fx["moe_t_e_score_correction_bias"],
             down=fx["moe_t_down_weight"], up=fx["moe_t_up_weight"],
             latent_norm=fx["moe_t_norm_weight"], sh1=fx["moe_t_shared_w1_weight"],
             sh3=fx["moe_t_shared_w3_weight"], sh2=fx["moe_t_shared_w2_weight"])
    for k, key in (("w1", "w1"), ("w3", "w3"), ("w2", "w2")):
        W[k] = np.concatenate([fx[f"moe_t_experts_{e}_{key}_weight"].ravel() for e in range(n)])
    return cfg, W, fx["moe_t_in"], fx["moe_t_out"]


def test_moe_latent_fixture(orc, fx):
    cfg, W, x, y = moe_fixture(fx)
    got = orc.moe_latent(x, cfg, W).reshape(y.shape)
    atol, rtol = float(fx["tol_abs"]), float(fx["tol_rel"])
    assert np.all(np.abs(got - y) <= atol + rtol * np.abs(y))


def test_oracle_reproduces_reference_goldens(orc, wl, gold):
    packed, scales, x = wl.gemv_inputs()
    assert np.array_equal(bits(orc.matmul_mxfp4(x, packed, scales, wl.HIDDEN, 2048)),
                          bits(gold["gemv_y"]))
    e0, xe = wl.expert(0), wl.expert_input()
    assert np.array_equal(bits(orc.expert_ffn(xe, e0, wl.HIDDEN, wl.INTER, act=1, wt=0.125)),
                          bits(gold["expert_silu"]))
    assert np.array_equal(bits(orc.expert_ffn(xe, e0, wl.HIDDEN, wl.INTER, act=0, wt=0.125)),
                          bits(gold["expert_situ"]))
    for name, pk, sc, xx, inn, rows, group in make_golden.edge_cases():
        assert np.array_equal(bits(orc.matmul_mxfp4(xx, pk, sc, inn, rows, group)),
                              bits(gold["edge_" + name])), name


def test_oracle_router_and_moe_goldens(orc, wl, gold):
    W = wl.router_weights()
    X = wl.tokens(64)
    for t in range(64):
        idx, w = orc.router(X[t], W, None, wl.TOPK)
        assert np.array_equal(idx, gold["router_idx"][t])
        assert np.array_equal(bits(w), bits(gold["router_wt"][t]))
    bank = wl.lazy_bank(gold["router_idx"][:8])
    out, idx, wt = orc.moe_routed(X[:8], W, None, bank, wl.HIDDEN, wl.INTER, wl.TOPK, act=1)
    assert np.array_equal(bits(out), bits(gold["moe8_out"]))


def test_gather_is_stable_expert_major(orc):
    rng = np.random.default_rng(5)
    idx = rng.integers(0, 40, (33, 8)).astype(np.int32)
    offsets, perm = orc.gather(idx, 40)
    flat = idx.ravel()
    want = sorted(range(flat.size), key=lambda a: (flat[a], a))
    assert perm.tolist() == want
    assert offsets[-1] == flat.size
    for e in range(40):
        assert offsets[e + 1] - offsets[e] == int((flat == e).sum())


def test_oracle_matches_compiled_reference_random(orc, ref):
    rng = np.random.default_rng(6)
    for rows, inn, group in ((70, 7168, 32), (33, 2048, 32), (19, 100, 20), (8, 64, 64)):
        pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
        sc = rng.integers(100, 140, rows * ((inn + group - 1) // group), dtype=np.uint8)
        x = rng.standard_normal(inn).astype(np.float32)
        assert np.array_equal(bits(orc.matmul_mxfp4(x, pk, sc, inn, rows, group)),
                              bits(ref.matmul_mxfp4(x, pk, sc, inn, rows, group)))
    W = rng.standard_normal((50, 300)).astype(np.float32)
    x = rng.standard_normal(300).astype(np.float32)
    b = rng.standard_normal(50).astype(np.float32) * 0.01
    i1, w1 = orc.router(x, W, b, 7)
    i2, w2 = ref.router(x, W, b, 7)
    assert np.array_equal(i1, i2) and np.array_equal(bits(w1), bits(w2))
    Wb = (rng.integers(0, 65536, (31, 257)).astype(np.uint16) & 0x7F7F)
    assert np.array_equal(bits(orc.matmul_bf16(x[:257], Wb)), bits(ref.matmul_bf16(x[:257], Wb)))


def test_nan_scale_group_skips_nonfinite_activations(orc, ref):
    """A group whose E8M0 byte is 255 is skipped whole (k3_ops.c:1478, 1536): an Inf or NaN
    activation inside it leaves the row finite, while one inside a group of a finite scale
    makes the row non-finite (0 * Inf = NaN, 1.5 * Inf = Inf). Oracle and compiled reference
    agree bit for bit; the rows that skip every non-finite activation equal the same GEMV
    with those activations set to zero."""
    rng = np.random.default_rng(255)
    rows, inn = 6, 128
    pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
    sc = rng.integers(120, 128, rows * inn // 32, dtype=np.uint8).reshape(rows, inn // 32)
    x = rng.standard_normal(inn).astype(np.float32)
    x[40], x[45] = np.inf, np.nan                    # both in group 1 (columns 32..63)
    sc[[0, 2, 5], 1] = 255                           # rows 0, 2, 5 skip group 1
    y = orc.matmul_mxfp4(x, pk, sc.ravel(), inn, rows)
    assert np.array_equal(bits(y), bits(ref.matmul_mxfp4(x, pk, sc.ravel(), inn, rows)))
    assert np.isfinite(y[[0, 2, 5]]).all() and not np.isfinite(y[[1, 3, 4]]).any()
    x0 = x.copy()
    x0[[40, 45]] = 0.0
    y0 = orc.matmul_mxfp4(x0, pk, sc.ravel(), inn, rows)
    assert np.array_equal(bits(y[[0, 2, 5]]), bits(y0[[0, 2, 5]]))


def test_q8_closed_form_matches_compiled_reference(ref):
    """k3_matmul_q8 (k3_ops.c:1221-1289) has no exactness contract (fp32 accumulation in the
    AVX2 reduction order): the compiled reference is within 1e-5 ||y||inf of the fp64 closed
    form (sum of int8 * x, then the row's scale), which the GPU test compares against; a
    row scale taken from the wrong end of the row would miss it by far."""
    from oracle import q8_exact, q8_rows
    rng = np.random.default_rng(8)
    for inn, out in ((7168, 96), (300, 17), (16, 3)):
        W, sc, q = q8_rows(rng, inn, out)
        x = rng.standard_normal(inn).astype(np.float32)
        want = q8_exact(x, sc, q)
        got = ref.matmul_q8(x, W, inn, out)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
        wrong = q8_exact(x, W[:, -4:].copy().view(np.float32).ravel(), q)
        assert np.abs(wrong - want).max() > 1e-2 * np.abs(want).max()


def test_expert_major_oracle_equals_per_token(orc, wl):
    """orc_expert_ffn_many (each expert dequantized once, all its tokens, the full-batch
    GPU tests' reference) equals orc_expert_ffn token by token bit for bit, and
    moe_outputs (expert-major, combine in slot order) equals orc_moe_routed's token-major
    loop on the same routing, bit for bit: the expert-major form only reorders the
    reference's operations."""
    rng = np.random.default_rng(5)
    for E, I, T in ((7168, 2048, 3), (1024, 512, 19)):
        ex = wl.expert(7, E, I)
        X = rng.standard_normal((T, E)).astype(np.float32)
        many = orc.expert_ffn_many(X, ex, E, I, act=1)
        one = np.stack([orc.expert_ffn(X[t], ex, E, I, act=1) for t in range(T)])
        assert np.array_equal(bits(many), bits(one))
        sit = orc.expert_ffn_many(X, ex, E, I, act=0)
        assert np.array_equal(bits(sit[0]), bits(orc.expert_ffn(X[0], ex, E, I, act=0)))
    E, I, N, K, T = 512, 256, 12, 3, 23
    bank = [wl.expert(e, E, I) for e in range(N)]
    W = (rng.standard_normal((N, E)) * 0.05).astype(np.float32)
    X = rng.standard_normal((T, E)).astype(np.float32)
    out, idx, wt = orc.moe_routed(X, W, None, bank, E, I, K)
    assert np.array_equal(bits(orc.moe_outputs(X, idx, wt, bank, E, I)), bits(out))
