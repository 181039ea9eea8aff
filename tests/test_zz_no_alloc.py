# SPDX-License-Identifier: Apache-2.0
"""k3d_moe_routed_static (no workspace argument, scratch in the library's static device
array) against k3d_moe_routed with a caller workspace, through the C ABI: two calls in a
row on the same layer, the second on a smaller batch, then a one-token call (the decode
path whose gate/up kernel selects the experts), each bit for bit equal to the workspace
form; a batch whose scratch exceeds the static array is refused with an error. At Kimi K3's
expert shape (3584 -> 3072 -> 3584, 896 experts, top-16) a 64-token decode batch fits the
array and gives the workspace form's bits."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
E, I, N, K = 7168, 2048, 64, 8


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def bank(gpu, wl):
    say("setup: 64-expert tiled bank at 7168 x 2048")
    b = gpu.DevBank([wl.expert(e) for e in range(N)], E, I, gpu.K3D_LAYOUT_TILED)
    yield b
    b.free()


def run(gpu, bank, X, W, static, want_perm, shape=(E, I, N, K)):
    L = gpu.lib()
    E, I, N, K = shape
    T = X.shape[0]
    bufs = {"x": gpu.DevBuf(X.nbytes).upload(X), "w": gpu.DevBuf(W.nbytes).upload(W),
            "out": gpu.DevBuf(T * E * 4), "idx": gpu.DevBuf(T * K * 4), "wt": gpu.DevBuf(T * K * 4),
            "perm": gpu.DevBuf(T * K * 4), "off": gpu.DevBuf((N + 1) * 4), "drops": gpu.DevBuf(4)}
    try:
        b = bufs
        perm = b["perm"].ptr if want_perm else None
        off = b["off"].ptr if want_perm else None
        args = (b["out"].ptr, b["idx"].ptr, b["wt"].ptr, b["x"].ptr, T, b["w"].ptr, None,
                bank.table.ptr, gpu.K3D_LAYOUT_TILED, E, I, N, K, 1, 1.0, gpu.K3_ACT_SILU, 4.0,
                25.0, 0)
        if static:
            rc = L.k3d_moe_routed_static(*args, perm, off, b["drops"].ptr, None)
            gpu.check(rc, "k3d_moe_routed_static")
        else:
            ws = gpu.DevBuf(L.k3d_moe_ws(T, E, I, N, K, 0))
            bufs["ws"] = ws
            gpu.check(L.k3d_moe_routed(*args, ws.ptr, ws.nbytes, perm, off, b["drops"].ptr, None),
                      "k3d_moe_routed")
        gpu.check(L.k3d_sync(None))
        res = [b["out"].download(np.empty((T, E), np.float32)),
               b["idx"].download(np.empty((T, K), np.int32)),
               b["wt"].download(np.empty((T, K), np.float32)),
               b["drops"].download(np.empty(1, np.int32))]
        if want_perm:
            res += [b["perm"].download(np.empty(T * K, np.int32)),
                    b["off"].download(np.empty(N + 1, np.int32))]
        return res
    finally:
        for v in bufs.values():
            v.free()


def same(a, b):
    assert len(a) == len(b)
    for u, v in zip(a, b):
        assert np.array_equal(np.ascontiguousarray(u).view(np.uint32),
                              np.ascontiguousarray(v).view(np.uint32))


def test_static_matches_workspace_form(gpu, wl, bank):
    L = gpu.lib()
    assert L.k3d_static_ws_bytes() == 40 << 20
    assert L.k3d_moe_ws(64, E, I, N, K, 0) <= L.k3d_static_ws_bytes()
    W = wl.router_weights(N, E, tag="noalloc.router")
    for T, perm in ((64, True), (5, False), (1, False)):
        say(f"case: static vs workspace T={T}")
        X = wl.tokens(T, E, tag=f"noalloc.x.{T}")
        got = run(gpu, bank, X, W, True, perm)
        want = run(gpu, bank, X, W, False, perm)
        same(got, want)
        assert got[3][0] == 0


def test_static_refuses_oversized_batch(gpu, wl, bank):
    say("case: static workspace too small")
    L = gpu.lib()
    T = 256
    assert L.k3d_moe_ws(T, E, I, N, K, 0) > L.k3d_static_ws_bytes()
    X = wl.tokens(T, E, tag="noalloc.x.big")
    W = wl.router_weights(N, E, tag="noalloc.router")
    bufs = [gpu.DevBuf(X.nbytes).upload(X), gpu.DevBuf(W.nbytes).upload(W),
            gpu.DevBuf(T * E * 4), gpu.DevBuf(T * K * 4), gpu.DevBuf(T * K * 4)]
    try:
        dx, dw, out, idx, wt = bufs
        rc = L.k3d_moe_routed_static(out.ptr, idx.ptr, wt.ptr, dx.ptr, T, dw.ptr, None, bank.table.ptr,
                                     gpu.K3D_LAYOUT_TILED, E, I, N, K, 1, 1.0, gpu.K3_ACT_SILU, 4.0,
                                     25.0, 0, None, None, None, None)
        assert rc != 0
        assert b"static workspace holds" in L.k3d_error()
    finally:
        for b in bufs:
            b.free()


def test_static_at_k3_shape(gpu, k3, wl):
    L = gpu.lib()
    shape = (3584, 3072, 896, 16)
    E3, I3, N3, K3 = shape
    assert L.k3d_moe_ws(64, E3, I3, N3, K3, 0) <= L.k3d_static_ws_bytes()
    say("setup: 896-entry tiled bank at 3584 x 3072, 64 experts present")
    experts = [k3.gen_expert(E3, I3, 61, e) if e < 64 else None for e in range(N3)]
    bank = gpu.DevBank(experts, E3, I3, gpu.K3D_LAYOUT_TILED)
    try:
        W = wl.router_weights(N3, E3, tag="noalloc.k3.router")
        for T in (64, 1):
            say(f"case: static vs workspace at the K3 shape, T={T}")
            X = wl.tokens(T, E3, tag=f"noalloc.k3.x.{T}")
            got = run(gpu, bank, X, W, True, T > 1, shape)
            want = run(gpu, bank, X, W, False, T > 1, shape)
            same(got, want)
    finally:
        bank.free()
