# SPDX-License-Identifier: Apache-2.0
"""The router and the routed layer at Kimi K3's real checkpoint shape (include/k3/k3.h:47-49,
95-99 of the reference): 896 experts, hidden 7168, top-16, renormalised weights scaled by
routed_scale, and an e_score_correction_bias that steers the selection only
(k3_ops.c:419-478). idx and weight bits equal the oracle's per-token router for every token,
at 1, 2, 4 (one kernel scores and certifies), 5, 64 and 4096 tokens (the fp64 matrix-core
partials); then the routed layer at the K3 expert shape (experts 3584 -> 3072 -> 3584,
SiTU-GLU) on an 896-expert tiled bank, routing bit-exact and outputs within 1e-4."""
import sys

import numpy as np
import pytest

from conftest import max_err_rel_inf

pytestmark = pytest.mark.gpu
N, HID, K, SCALE = 896, 7168, 16, 2.827


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def router(wl):
    W = wl.router_weights(N, HID, tag="k3.router")
    bias = wl.k3amd.gen_normal(N, wl.stream("k3.router.bias"), 0.0, 0.02)
    return W, bias


@pytest.mark.parametrize("T", [1, 2, 4, 5, 64, 4096])
def test_router_k3_shape(gpu, orc, wl, router, T):
    say(f"case: router 896x7168 top-16 biased, T={T}")
    W, bias = router
    X = wl.tokens(T, HID, tag=f"k3.router.x.{T}")
    idx, wt = gpu.router_device(X, W, bias, K, 1, SCALE)
    say(f"  recomputed logits: {int(gpu.router_device.recomputed.sum())}")
    changed = 0
    for t in range(T):
        i2, w2 = orc.router(X[t], W, bias, K, 1, SCALE)
        assert np.array_equal(idx[t], i2), t
        assert np.array_equal(bits(wt[t]), bits(w2)), t
        if t < 64:
            i0, _ = orc.router(X[t], W, None, K, 1, SCALE)
            changed += not np.array_equal(np.sort(i0), np.sort(i2))
    assert changed > 0 or T < 4          # the bias reorders the selection


def test_router_k3_shape_host_api(gpu, orc, wl, router):
    """k3_router, the reference's own single-token entry point, at the same shape."""
    say("case: k3_router host API 896x7168")
    W, bias = router
    X = wl.tokens(3, HID, tag="k3.router.host")
    for t in range(3):
        i1, w1 = gpu.router(X[t], W, bias, K, 1, SCALE)
        i2, w2 = orc.router(X[t], W, bias, K, 1, SCALE)
        assert np.array_equal(i1, i2) and np.array_equal(bits(w1), bits(w2))


@pytest.fixture(scope="module")
def k3bank(gpu, wl):
    say("setup: 896-expert tiled bank of 3584 x 3072 experts (15.7 GB)")

    class Lazy:
        def __len__(self):
            return N

        def __iter__(self):
            for e in range(N):
                yield wl.expert(e, 3584, 3072)
    b = gpu.DevBank(Lazy(), 3584, 3072, gpu.K3D_LAYOUT_TILED)
    yield b
    b.free()


@pytest.mark.parametrize("T", [1, 4, 64])
def test_routed_layer_k3_expert_shape(gpu, orc, wl, k3bank, T):
    say(f"case: routed layer 896 experts 3584x3072 top-16 SiTU, T={T}")
    W = wl.router_weights(N, 3584, tag="k3.latent.router")
    bias = wl.k3amd.gen_normal(N, wl.stream("k3.latent.bias"), 0.0, 0.02)
    X = wl.tokens(T, 3584, tag=f"k3.latent.x.{T}")
    out, idx, wt, perm, off, drops = gpu.moe_routed_device(
        k3bank, X, W, bias, K, 1, SCALE, act=gpu.K3_ACT_SITU, prec=0, hidden=3584, inter=3072,
        want_perm=T > 4)
    bank = wl.lazy_bank(idx, N, 3584, 3072)
    o2, i2, w2 = orc.moe_routed(X, W, bias, bank, 3584, 3072, K, 1, SCALE, act=0)
    assert np.array_equal(idx, i2)
    assert np.array_equal(bits(wt), bits(w2))
    assert drops == 0
    if perm is not None:
        o_, p_ = orc.gather(idx, N)
        assert np.array_equal(off, o_) and np.array_equal(perm, p_)
    for t in range(T):
        assert max_err_rel_inf(out[t], o2[t]) <= 1e-4, t
