# SPDX-License-Identifier: Apache-2.0
"""k3_moe / k3_moe_prefill with MXFP4 experts streamed through a K3ExpertSrc, at Kimi K3's
expert shapes (hidden 7168, latent 3584, moe_inter 3072, top-16, 2 shared experts, bf16
trunk), against the oracle's restatement of the reference (orc_moe_q, itself pinned bit for
bit to the compiled reference in test_oracle_moe_q.py).

Per case: idx/wt bit-exact (what the reference leaves in them), k3_expert_drops equal, the
source sees the reference's exact get / getmany / resident sequence, and
max|out - ref| <= 1e-4 * ||ref||inf. Token counts cross the prefill's 64-token chunk (65 =
64 + 1, 130 = 64 + 64 + 2). Also: one expert whose get() fails, the cache-only draft
routing, and the library's HBM bank (k3_devbank_*) as the source, filled through an
upstream source or from the reference's on-disk expert runs, with no weight bytes moved
once resident."""
import sys

import numpy as np
import pytest

from conftest import max_err_rel_inf
from oracle import PySource, oracle_moe_q

pytestmark = pytest.mark.gpu
TOL = 1e-4
N_EXPERTS, TOPK = 40, 16


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def k3layer(wl):
    say("setup: K3-shape LatentMoE layer (40 experts of 3584 x 3072)")
    return wl.latent_layer(7168, 3584, 3072, N_EXPERTS, TOPK, tag="gpuq.k3")


def tokens(wl, T):
    return wl.tokens(T, 7168, tag=f"gpuq.x.{T}")


def compare(got, want, check_calls=True):
    (o1, i1, w1, d1, c1), (o2, i2, w2, d2, c2) = got, want
    assert np.array_equal(i1, i2)
    assert np.array_equal(bits(w1), bits(w2))
    assert d1 == d2
    if check_calls:
        assert c1 == c2
    err = max_err_rel_inf(o1, o2)
    assert err <= TOL, err


def run_pair(gpu, orc, layer, x, prefill, fail=(), resident=None, cache_only=0, layer_id=5):
    cfg, W, experts = layer
    s1 = PySource(experts, fail=fail, resident=resident)
    got = gpu.moe(x, cfg, W, 1, s1.ptr, prefill, layer=layer_id, cache_only=cache_only)
    s2 = PySource(experts, fail=fail, resident=resident)
    want = oracle_moe_q(orc, x, cfg, W, 1, s2, prefill, layer=layer_id, cache_only=cache_only)
    return got + (s1.calls,), want + (s2.calls,)


@pytest.mark.parametrize("T", [1, 3, 65])
def test_k3_moe_streamed(gpu, orc, wl, k3layer, T):
    say(f"case: k3_moe streamed T={T}")
    got, want = run_pair(gpu, orc, k3layer, tokens(wl, T), 0)
    compare(got, want)


@pytest.mark.parametrize("T", [1, 3, 64, 65, 130])
def test_k3_moe_prefill_streamed(gpu, orc, wl, k3layer, T):
    say(f"case: k3_moe_prefill streamed T={T}")
    got, want = run_pair(gpu, orc, k3layer, tokens(wl, T), 1)
    compare(got, want)


def _victim(orc, layer, x):
    cfg, W, _ = layer
    idx = np.stack([orc.router(x[t], W["gate"], W["bias"], cfg["topk"])[0] for t in range(len(x))])
    return int(np.bincount(idx.ravel()).argmax())


@pytest.mark.parametrize("T,prefill", [(3, 0), (130, 1), (65, 1)])
def test_k3_moe_failed_fetch(gpu, orc, wl, k3layer, T, prefill):
    """get() fails for the most popular expert: drops per (token, slot) in k3_moe, per
    64-token chunk in k3_moe_prefill, and the slots contribute nothing."""
    say(f"case: k3_moe failed fetch T={T} prefill={prefill}")
    x = tokens(wl, T)
    v = _victim(orc, k3layer, x)
    got, want = run_pair(gpu, orc, k3layer, x, prefill, fail={v})
    assert want[3] > 0
    compare(got, want)


@pytest.mark.parametrize("prefill", [0, 1])
def test_k3_moe_cache_only(gpu, orc, wl, k3layer, prefill):
    """Draft routing among the resident experts (every other id): idx compacted in place
    with the router's values left in the tail, weights renormalised over the kept slots."""
    say(f"case: k3_moe cache_only prefill={prefill}")
    got, want = run_pair(gpu, orc, k3layer, tokens(wl, 4), prefill, cache_only=1,
                         resident=set(range(0, N_EXPERTS, 2)))
    compare(got, want)
    assert not any(c[0] == "get" for c in got[4])


@pytest.mark.parametrize("layout", [0, 1])
def test_k3_moe_hbm_bank_upstream(gpu, orc, wl, k3layer, layout):
    """The HBM bank in front of a host source: the first call admits each expert once over
    PCIe, a second call on other tokens moves no weight bytes for experts already resident,
    and both match the oracle."""
    say(f"case: k3_moe HBM bank over an upstream source, layout {layout}")
    cfg, W, experts = k3layer
    up = PySource(experts)
    bank = gpu.HbmBank(2, N_EXPERTS, 3584, 3072, N_EXPERTS, layout, up.ptr)
    try:
        x = tokens(wl, 65)
        got = gpu.moe(x, cfg, W, 1, bank.src, 1, layer=1)
        want = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts), 1, layer=1)
        compare(got + ([],), want + ([],), check_calls=False)
        st1 = bank.stats()
        used = {e for e in range(N_EXPERTS) if ("get", 1, e) in up.calls}
        assert st1["misses"] == len(used) == st1["resident"]
        assert st1["bytes_uploaded"] == len(used) * gpu.lib().k3_devbank_run_bytes(3584, 3072)
        # another batch: only the experts not yet resident cross PCIe
        x2 = tokens(wl, 3)
        st_before = bank.stats()
        got2 = gpu.moe(x2, cfg, W, 1, bank.src, 0, layer=1)
        want2 = oracle_moe_q(orc, x2, cfg, W, 1, PySource(experts), 0, layer=1)
        compare(got2 + ([],), want2 + ([],), check_calls=False)
        st2 = bank.stats()
        idx2 = np.stack([orc.router(x2[t], W["gate"], W["bias"], TOPK)[0] for t in range(3)])
        new = {int(e) for e in idx2.ravel()} - used
        assert st2["bytes_uploaded"] - st_before["bytes_uploaded"] == \
            len(new) * gpu.lib().k3_devbank_run_bytes(3584, 3072)
        # the same tokens again: all resident, zero bytes
        st3 = bank.stats()
        got3 = gpu.moe(x2, cfg, W, 1, bank.src, 0, layer=1)
        assert bank.stats()["bytes_uploaded"] == st3["bytes_uploaded"]
        assert np.array_equal(bits(got3[0]), bits(got2[0]))
    finally:
        bank.destroy()


def test_k3_moe_hbm_bank_from_runs(gpu, orc, wl, k3layer):
    """Experts admitted from the reference's contiguous on-disk run (w1.p w1.s w2.p w2.s
    w3.p w3.s, 17,547,264 bytes), no upstream source; one expert never admitted counts as a
    failed fetch."""
    say("case: k3_moe HBM bank from on-disk runs")
    cfg, W, experts = k3layer
    assert gpu.lib().k3_devbank_run_bytes(3584, 3072) == 17547264
    bank = gpu.HbmBank(1, N_EXPERTS, 3584, 3072, N_EXPERTS, 1, None)
    try:
        x = tokens(wl, 130)
        missing = _victim(orc, k3layer, x)
        for e, ex in experts.items():
            if e != missing:
                bank.put_run(0, e, wl.expert_run(ex))
        with pytest.raises(RuntimeError):
            bank.put_run(0, 0, wl.expert_run(experts[0])[:-1])
        st0 = bank.stats()
        got = gpu.moe(x, cfg, W, 1, bank.src, 1, layer=0)
        want = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts, fail={missing}), 1, layer=0)
        assert want[3] > 0
        compare(got + ([],), want + ([],), check_calls=False)
        assert bank.stats()["bytes_uploaded"] == st0["bytes_uploaded"]
    finally:
        bank.destroy()


def test_k3_moe_hbm_bank_eviction(gpu, orc, wl, k3layer):
    """A bank of 20 slots for 40 experts: one-token calls evict least recently used experts
    and stay exact."""
    say("case: k3_moe HBM bank eviction")
    cfg, W, experts = k3layer
    up = PySource(experts)
    bank = gpu.HbmBank(1, N_EXPERTS, 3584, 3072, 20, 1, up.ptr)
    try:
        for t in range(4):
            x = wl.tokens(1, 7168, tag=f"gpuq.evict.{t}")
            got = gpu.moe(x, cfg, W, 1, bank.src, 0)
            want = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts), 0)
            compare(got + ([],), want + ([],), check_calls=False)
        st = bank.stats()
        assert st["resident"] <= 20 and st["evictions"] > 0
    finally:
        bank.destroy()


@pytest.mark.parametrize("slots,T,prefill", [(20, 3, 0), (20, 3, 1), (20, 65, 1), (10, 2, 0), (10, 2, 1)])
def test_k3_moe_hbm_bank_overflow(gpu, orc, wl, k3layer, slots, T, prefill):
    """One call naming more distinct experts than the bank has slots: several tokens at
    top-16 over 20 slots (between tokens, or inside a 64-token chunk), and 10 slots, fewer
    than one token's 16 experts. The call computes what it has fetched, releases its slots
    and goes on: no drops, no failed admissions, the oracle's result."""
    say(f"case: k3_moe HBM bank of {slots} slots, T={T} prefill={prefill}")
    cfg, W, experts = k3layer
    up = PySource(experts)
    bank = gpu.HbmBank(1, N_EXPERTS, 3584, 3072, slots, 1, up.ptr)
    try:
        x = wl.tokens(T, 7168, tag=f"gpuq.overflow.{T}")
        idx = np.stack([orc.router(x[t], W["gate"], W["bias"], TOPK)[0] for t in range(T)])
        assert len(set(idx.ravel().tolist())) > slots
        got = gpu.moe(x, cfg, W, 1, bank.src, prefill)
        want = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts), prefill)
        assert want[3] == 0
        compare(got + ([],), want + ([],), check_calls=False)
        st = bank.stats()
        assert st["failures"] == 0 and st["resident"] <= slots
    finally:
        bank.destroy()


def test_k3_moe_threads(gpu, orc, wl, k3layer):
    """Two host threads calling the library at once (the reference's kernels are
    re-entrant): each result equals the one computed alone."""
    say("case: k3_moe from two threads")
    import threading
    cfg, W, experts = k3layer
    xs = [tokens(wl, 3), tokens(wl, 1)]
    alone = [gpu.moe(x, cfg, W, 1, PySource(experts).ptr, 1)[0] for x in xs]
    res = [None, None]
    srcs = [PySource(experts), PySource(experts)]

    def work(i):
        res[i] = gpu.moe(xs[i], cfg, W, 1, srcs[i].ptr, 1)[0]
    th = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for i in range(2):
        assert np.array_equal(bits(res[i]), bits(alone[i]))
