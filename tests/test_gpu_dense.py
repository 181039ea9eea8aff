# SPDX-License-Identifier: Apache-2.0
"""Dense bf16 / fp32 GEMV and GEMM (the trunk projections and the dense shared expert)
through the C ABI against the oracle's k3_matmul_bf16 / k3_matmul restatement (fp64
accumulation, src/core/k3_ops.c:265-291, 1108-1213 of the reference):
max|err| <= 1e-4 ||ref||inf for fp32 activations; k3_matmul_bf16 bit-identical to
k3_matmul on the widened weights for one token (the reference's own invariant,
tests/unit/test_ops.c:811-848)."""
import sys

import numpy as np
import pytest

from conftest import max_err_rel_inf

pytestmark = pytest.mark.gpu
TOL = 1e-4


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def dev_matmul(gpu, X, W, bf16=True):
    L = gpu.lib()
    X = np.ascontiguousarray(X, np.float32)
    T, inn = X.shape
    out = W.shape[0]
    bufs = [gpu.DevBuf(X.nbytes).upload(X), gpu.DevBuf(W.nbytes).upload(W), gpu.DevBuf(T * out * 4)]
    try:
        dx, dw, dy = bufs
        fn = L.k3d_matmul_bf16 if bf16 else L.k3d_matmul_f32
        gpu.check(fn(dy.ptr, dx.ptr, T, dw.ptr, inn, out, None), "k3d_matmul")
        gpu.check(L.k3d_sync(None))
        return dy.download(np.empty((T, out), np.float32))
    finally:
        for b in bufs:
            b.free()


def test_trunk_gemv_bench_shape(gpu, orc, k3):
    """The reference benchmark's bf16 GEMV (KDA q-projection 7168 -> 12288) with its own
    inputs: within tolerance of the oracle, whose output hashes to the reference's."""
    say("case: bf16 gemv 12288x7168, bench inputs")
    W = orc.fill_bf16(7168 * 12288, 12345).reshape(12288, 7168)
    x = orc.fill_f(7168, 999)
    want = orc.matmul_bf16(x, W)
    assert orc.fnv1a(want) == 0x83C8504A4CB3FAC6
    assert max_err_rel_inf(gpu.matmul_bf16(x, W), want) <= TOL
    assert max_err_rel_inf(dev_matmul(gpu, x[None], W)[0], want) <= TOL


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8, 17])
@pytest.mark.parametrize("shape", [(3584, 7168), (7168, 6144), (100, 264), (257, 72)])
def test_dense_matmul_tokens(gpu, orc, k3, T, shape):
    out, inn = shape
    say(f"case: bf16/f32 matmul {out}x{inn} T={T}")
    Wb = k3.gen_bf16_normal(inn * out, 71 + T, 0.0, 0.02).reshape(out, inn)
    X = k3.gen_normal(T * inn, 72 + T).reshape(T, inn)
    Y = dev_matmul(gpu, X, Wb)
    Wf = (Wb.astype(np.uint32) << 16).view(np.float32)
    Yf = dev_matmul(gpu, X, Wf, bf16=False)
    for t in range(T):
        want = orc.matmul_bf16(X[t], Wb)
        assert max_err_rel_inf(Y[t], want) <= TOL, t
        assert max_err_rel_inf(Yf[t], want) <= TOL, t
    if T == 1:
        assert np.array_equal(bits(Y), bits(Yf))


@pytest.mark.parametrize("T,prec", [(512, 1), (512, 0), (77, 0), (130, 1)])
def test_shared_expert_config4_shape(gpu, orc, wl, T, prec):
    """The dense SwiGLU shared expert at 7168 -> 2048 -> 7168 on the matrix cores, added
    onto an existing output (the reference's ot[i] += sdn[i]): sampled tokens against the
    oracle's bf16 composition (k3_matmul_bf16, SiLU-GLU, k3_matmul_bf16)."""
    say(f"case: shared expert 7168/2048 T={T} prec={prec}")
    E, I = 7168, 2048
    w1, w3, w2 = wl.shared_expert_weights()
    X = wl.tokens(T, tag=f"dense.shared.{T}")
    y0 = wl.tokens(T, tag=f"dense.shared.y0.{T}") * 0.5
    got = gpu.shared_expert_device(X, w1, w3, w2, E, I, prec=prec, y0=y0)
    tol = TOL if prec == 0 else 2e-2
    for t in np.random.default_rng(T).choice(T, min(T, 12), replace=False):
        g = orc.matmul_bf16(X[t], w1.reshape(I, E))
        u = orc.matmul_bf16(X[t], w3.reshape(I, E))
        s = orc.matmul_bf16(orc.silu_glu(np.concatenate([g, u]), I), w2.reshape(E, I))
        want = y0[t] + s
        assert max_err_rel_inf(got[t], want) <= tol, t
        assert max_err_rel_inf(got[t] - y0[t], s) <= (tol if prec == 0 else 2e-2), t


@pytest.mark.parametrize("inn,out", [(7168, 3584), (300, 17), (16, 3)])
def test_matmul_q8(gpu, k3, inn, out):
    """k3_matmul_q8 (the draft model's int8 rows, k3_mmw's K3_WI8 branch; reference
    k3_ops.c:1221-1289, no exactness contract there): within 1e-4 ||ref||inf of the fp64
    closed form, which the compiled reference matches to 1e-5 (tests/test_oracle.py), and
    of the compiled reference itself where it is built."""
    from oracle import Ref, q8_exact, q8_rows
    say(f"case: k3_matmul_q8 {out}x{inn}")
    rng = np.random.default_rng(inn + out)
    W, sc, q = q8_rows(rng, inn, out)
    x = rng.standard_normal(inn).astype(np.float32)
    got = k3.matmul_q8(x, W, inn, out)
    assert max_err_rel_inf(got, q8_exact(x, sc, q)) <= TOL
    if Ref.available():
        assert max_err_rel_inf(got, Ref().matmul_q8(x, W, inn, out)) <= TOL


@pytest.mark.parametrize("T", [1, 4])
def test_trunk_o_projection(gpu, orc, T):
    """The KDA/MLA o-projection shape (12288 -> 7168, bf16) through k3_matmul_bf16 and the
    device entry, against the oracle."""
    say(f"case: bf16 gemv 7168x12288 (o-projection), T={T}")
    W = orc.fill_bf16(12288 * 7168, 4321).reshape(7168, 12288)
    X = np.stack([orc.fill_f(12288, 50 + t) for t in range(T)])
    want = np.stack([orc.matmul_bf16(X[t], W) for t in range(T)])
    got = dev_matmul(gpu, X, W)
    for t in range(T):
        assert max_err_rel_inf(got[t], want[t]) <= TOL, t
    assert max_err_rel_inf(gpu.matmul_bf16(X[0], W), want[0]) <= TOL
