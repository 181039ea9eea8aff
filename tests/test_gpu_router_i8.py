# SPDX-License-Identifier: Apache-2.0
"""The router's chunk partials of many tokens on the int8 matrix cores (k3_route_i8.hip):
every row split into exact int8 digits under one power-of-two scale per chunk, the digit
products summed exactly in int32 per level, and a bound R_k on what the left-out digits
can change. The certification (router_final_kernel) relies on two facts per (chunk k,
token t, expert e):

    |P_k - exact chunk sum| <= 2^-53 R_k   and   R_k >= sum_i |exact prefix sum at column i|,

checked here against the chunk sums and prefixes in extended precision, on rows that take
every branch of the split: rows whose largest value is 128 or more (scaled down, small
values may lose bits to the subnormal range), zero rows, values spread over many binades
(left-out remainders), tiny and subnormal values, and a non-finite value (its chunk falls
back to a plain fp64 chain). idx and weight bits equal the oracle's per-token router
(k3_ops.c:419-478) for every token. The int8 partials serve 1024 tokens and more; the fp64
matrix-core partials of fewer tokens are held to the same contract."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HID = 7168


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def special_inputs(T, N, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, HID)) * 0.02).astype(np.float32)
    X = rng.standard_normal((T, HID)).astype(np.float32)
    X[0, 5] = 1500.0                                   # chunk 0 scaled down
    X[1] = 0.0                                         # a zero row
    X[2, : HID // 2] *= np.float32(1e-30)              # tiny values in half the row
    X[3] *= np.exp2(rng.integers(-40, 8, HID)).astype(np.float32)   # many binades
    X[4, 100:200] = np.float32(1e-41)                  # subnormal values
    X[5, 3000] = np.inf                                # a non-finite value
    W[7, 64] = 900.0
    W[8] = 0.0
    W[9] = (rng.standard_normal(HID) * 1e-37).astype(np.float32)
    W[10] *= np.exp2(rng.integers(-30, 4, HID)).astype(np.float32)
    return W, X


def check_contract(part, rb, chunk, W, X, tokens):
    """|P - exact| <= 2^-53 R and R >= sum |exact prefix| for the finite rows in `tokens`"""
    ks = part.shape[0]
    Wl = W.astype(np.longdouble)
    worst_err = worst_pre = 0.0
    for t in tokens:
        if not np.isfinite(X[t]).all():
            continue
        prod = Wl * X[t].astype(np.longdouble)[None, :]          # exact in fp64, kept in 80 bits
        for k in range(ks):
            seg = prod[:, k * chunk:min(HID, (k + 1) * chunk)]
            pre = np.cumsum(seg, axis=1)
            exact = pre[:, -1]
            abs_sum = np.abs(seg).sum(axis=1)
            # the extended-precision sums err by at most n 2^-64 of sum |products|
            slack = abs_sum * seg.shape[1] * np.longdouble(2.0) ** -63
            err = np.abs(part[k, t].astype(np.longdouble) - exact)
            lim = rb[k, t].astype(np.longdouble) * np.longdouble(2.0) ** -53 + slack
            ratio = err / np.where(lim > 0, lim, 1)
            assert np.all(err <= lim), (t, k, int(np.argmax(ratio)), float(ratio.max()))
            worst_err = max(worst_err, float(ratio.max()))
            spre = np.abs(pre).sum(axis=1)
            ok = rb[k, t].astype(np.longdouble) >= spre * (1 - np.longdouble(2.0) ** -40)
            assert np.all(ok), (t, k, int(np.argmin(rb[k, t] / np.maximum(spre, 1e-300))))
            with np.errstate(divide="ignore", invalid="ignore"):
                q = np.where(rb[k, t] > 0, spre / rb[k, t].astype(np.longdouble), 0)
            worst_pre = max(worst_pre, float(q.max()))
    return worst_err, worst_pre


@pytest.mark.parametrize("T,N,K", [(1030, 384, 8), (1100, 200, 6)])
def test_router_i8_partials_and_selection(gpu, orc, T, N, K):
    say(f"case: int8 router partials T={T} N={N} K={K}")
    W, X = special_inputs(T, N, T + N)
    idx, wt = gpu.router_device(X, W, None, K, partials=True)
    part, rb, chunk = gpu.router_device.partials
    say(f"  chunk {chunk} ({part.shape[0]} chunks), recomputed logits: "
        f"{int(gpu.router_device.recomputed.sum())}")
    assert chunk % 256 == 0
    assert gpu.router_device.recomputed.sum() <= max(4, T // 64)
    tokens = list(range(12)) + list(range(T - 20, T))
    e, p = check_contract(part, rb, chunk, W, X, tokens)
    say(f"  worst |P - exact| / (2^-53 R): {e:.3g}; worst sum|prefix| / R: {p:.3g}")
    assert np.isnan(part[:, 5]).any() or np.isinf(part[:, 5]).any()   # the non-finite row
    for t in range(T):
        i2, w2 = orc.router(X[t], W, None, K)
        assert np.array_equal(idx[t], i2), t
        assert np.array_equal(bits(wt[t]), bits(w2)), t


@pytest.mark.parametrize("T,N", [(300, 384), (64, 200)])
def test_router_fp64_partials_contract(gpu, orc, T, N):
    """The same contract for the fp64 matrix-core partials that serve 5 to 1023 tokens
    (router_partial_mfma_kernel, k3_route.hip), on the same special rows: the chunk sums
    within 2^-53 R_k of the exact ones, R_k above the exact prefix magnitudes, and idx /
    weight bits equal to the oracle's."""
    say(f"case: fp64 router partials T={T} N={N}")
    W, X = special_inputs(T, N, 7 * T + N)
    idx, wt = gpu.router_device(X, W, None, 8, partials=True)
    part, rb, chunk = gpu.router_device.partials
    say(f"  chunk {chunk} ({part.shape[0]} chunks), recomputed logits: "
        f"{int(gpu.router_device.recomputed.sum())}")
    e, p = check_contract(part, rb, chunk, W, X, list(range(12)) + [T - 1])
    say(f"  worst |P - exact| / (2^-53 R): {e:.3g}; worst sum|prefix| / R: {p:.3g}")
    for t in range(T):
        i2, w2 = orc.router(X[t], W, None, 8)
        assert np.array_equal(idx[t], i2), t
        assert np.array_equal(bits(wt[t]), bits(w2)), t


def test_router_i8_biased_top16(gpu, orc):
    """896 experts (14 expert tiles), top-16 with a selection bias and routed scale, 1030
    tokens: idx and weight bits equal the oracle's for every token."""
    say("case: int8 router partials T=1030 N=896 K=16 biased")
    rng = np.random.default_rng(77)
    W = (rng.standard_normal((896, HID)) * 0.02).astype(np.float32)
    X = rng.standard_normal((1030, HID)).astype(np.float32)
    bias = (rng.standard_normal(896) * 0.02).astype(np.float32)
    idx, wt = gpu.router_device(X, W, bias, 16, 1, 2.827, partials=True)
    part, rb, chunk = gpu.router_device.partials
    say(f"  chunk {chunk}, recomputed logits: {int(gpu.router_device.recomputed.sum())}")
    check_contract(part, rb, chunk, W, X, [0, 1, 1029])
    for t in range(1030):
        i2, w2 = orc.router(X[t], W, bias, 16, 1, 2.827)
        assert np.array_equal(idx[t], i2), t
        assert np.array_equal(bits(wt[t]), bits(w2)), t
