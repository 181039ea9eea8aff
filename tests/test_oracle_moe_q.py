# SPDX-License-Identifier: Apache-2.0
"""Pins the oracle's streamed-expert LatentMoE (orc_moe_q) to the compiled reference's own
k3_moe and k3_moe_prefill (src/core/k3_ops.c:556-825), driven through one K3ExpertSrc:
outputs, idx/wt and k3_expert_drops bit for bit, and the exact sequence of get / getmany /
resident calls the reference makes. Cases cross the prefill's 64-token chunk (65 = 64 + 1,
130 = 64 + 64 + 2), include a source whose get() fails for one expert, the cache-only draft
routing, and a source without getmany / resident. CPU only."""
import numpy as np
import pytest

from oracle import PySource, oracle_moe_q, ref_moe_q

SMALL = dict(hidden=256, latent=128, inter=96, n_experts=12, topk=4, n_shared=2)


@pytest.fixture(scope="module")
def layer(wl):
    return wl.latent_layer(**SMALL, tag="orcq.small")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run_both(orc, ref, layer, wl, T, prefill, fail=(), resident=None, cache_only=0,
             with_getmany=True, with_resident=True, bias=True):
    cfg, W, experts = layer
    W = dict(W) if bias else dict(W, bias=None)
    x = wl.tokens(T, cfg["hidden"], tag=f"orcq.x.{T}")
    res = []
    for fn in (ref_moe_q, oracle_moe_q):
        src = PySource(experts, fail=fail, resident=resident, with_getmany=with_getmany,
                       with_resident=with_resident)
        out, idx, wt, drops = fn(ref if fn is ref_moe_q else orc, x, cfg, W, 1, src, prefill,
                                 layer=3, cache_only=cache_only)
        res.append((out, idx, wt, drops, src.calls))
    return res


def assert_same(r_ref, r_orc):
    (o1, i1, w1, d1, c1), (o2, i2, w2, d2, c2) = r_ref, r_orc
    assert np.array_equal(bits(o1), bits(o2))
    assert np.array_equal(i1, i2)
    assert np.array_equal(bits(w1), bits(w2))
    assert d1 == d2
    assert c1 == c2


@pytest.mark.parametrize("T", [1, 3, 65])
def test_moe_q_tokens_matches_reference(orc, ref, wl, layer, T):
    r = run_both(orc, ref, layer, wl, T, prefill=0)
    assert_same(*r)
    assert r[0][3] == 0


@pytest.mark.parametrize("T", [1, 3, 65, 130])
def test_moe_q_prefill_matches_reference(orc, ref, wl, layer, T):
    r = run_both(orc, ref, layer, wl, T, prefill=1)
    assert_same(*r)


@pytest.mark.parametrize("prefill", [0, 1])
@pytest.mark.parametrize("T", [3, 65, 130])
def test_moe_q_failed_fetch(orc, ref, wl, layer, T, prefill):
    """One expert's get() fails: per (token, slot) drops in k3_moe, one per 64-token chunk
    that holds it in k3_moe_prefill."""
    cfg = layer[0]
    x = wl.tokens(T, cfg["hidden"], tag=f"orcq.x.{T}")
    idx_all = np.stack([orc.router(x[t], layer[1]["gate"], layer[1]["bias"], cfg["topk"])[0]
                        for t in range(T)])
    victim = int(np.bincount(idx_all.ravel()).argmax())
    r = run_both(orc, ref, layer, wl, T, prefill=prefill, fail={victim})
    assert_same(*r)
    per_slot = int((idx_all == victim).sum())
    if prefill and T > 1:
        chunks = [idx_all[t0:t0 + 64] for t0 in range(0, T, 64)]
        want = sum((int((c == victim).sum()) if len(c) == 1 else int((c == victim).any()))
                   for c in chunks)
    else:
        want = per_slot
    assert r[0][3] == want > 0


@pytest.mark.parametrize("T", [1, 4])
def test_moe_q_cache_only(orc, ref, wl, layer, T):
    """Draft routing over the resident subset: idx compacted in place, weights renormalised
    over the kept slots, nothing read through get()."""
    r = run_both(orc, ref, layer, wl, T, prefill=1, cache_only=1, resident=set(range(0, 12, 2)))
    assert_same(*r)
    assert not any(c[0] == "get" for c in r[0][4])


def test_moe_q_without_optional_callbacks(orc, ref, wl, layer):
    r = run_both(orc, ref, layer, wl, 5, prefill=1, with_getmany=False, with_resident=False,
                 bias=False)
    assert_same(*r)


def test_moe_q_prefill_equals_per_token(orc, wl, layer):
    """The reference's own claim (k3_ops.c:677-681): the expert-major batch gives every token
    the same bits as the per-token form."""
    cfg, W, experts = layer
    x = wl.tokens(70, cfg["hidden"], tag="orcq.x.70")
    a = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts), 1)[0]
    b = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts), 0)[0]
    assert np.array_equal(bits(a), bits(b))


def test_moe_q_fp32_trunk_matches_latent_fixture_path(orc, ref, wl, layer):
    """wdt 0 (fp32 trunk) through the same source."""
    cfg, W, experts = layer
    Wf = dict(W)
    for k in ("down", "up", "sh1", "sh3", "sh2"):
        Wf[k] = (W[k].astype(np.uint32) << 16).view(np.float32)
    x = wl.tokens(3, cfg["hidden"], tag="orcq.x.3")
    r1 = ref_moe_q(ref, x, cfg, Wf, 0, PySource(experts), 0)
    r2 = oracle_moe_q(orc, x, cfg, Wf, 0, PySource(experts), 0)
    b1 = oracle_moe_q(orc, x, cfg, W, 1, PySource(experts), 0)
    assert np.array_equal(bits(r1[0]), bits(r2[0]))
    assert np.array_equal(bits(r2[0]), bits(b1[0]))   # bf16 = fp32 on the widened weights
