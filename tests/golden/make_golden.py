# SPDX-License-Identifier: Apache-2.0
"""Writes the golden fixtures under tests/golden/. Run in a container that has the
reference tree at /root/reference (read-only) and oracle/_ref built from it.

  ref_fixtures.npz   the reference's own hot-path fixtures, converted from JSON to arrays
                     (data only): tests/fixtures/mxfp4.json, ops/router.json,
                     ops/situ_glu.json, ops/rmsnorm.json, ops/moe.json, and the tolerance of
                     ops/MANIFEST.json
  ref_golden.npz     outputs of the COMPILED reference (oracle/_ref, built from the
                     reference's src/core/k3_ops.c) on this project's workloads: the
                     2048x7168 GEMV, one expert (SiLU and SiTU), the 384x7168 top-8 router
                     over 64 tokens, 8 tokens of the 384-expert MoE layer, and MXFP4 edge
                     cases (scale bytes 0/1/254/255, ragged shapes, group 16)

usage: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REF = "/root/reference/tests/fixtures"
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "kimi-k3-in-c_amd"))

from oracle import Ref  # noqa: E402
import workloads as wl  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def arr(d, dtype=np.float32):
    return np.asarray(d["data"], dtype=np.float64).astype(dtype).reshape(d["shape"])


def convert_reference_fixtures():
    out = {}
    m = json.load(open(os.path.join(REF, "mxfp4.json")))
    out["mx_packed"] = arr(m["packed"], np.uint8)
    out["mx_scales"] = arr(m["scales"], np.uint8)
    out["mx_expected"] = arr(m["expected"])
    out["mx_swapped_first64"] = np.asarray(m["expected_swapped_nibbles"]["first64"], np.float32)
    out["mx_group"] = np.int32(m["group_size"])
    r = json.load(open(os.path.join(REF, "ops", "router.json")))
    out["rt_W"] = arr(r["gate_weight"])
    out["rt_bias"] = arr(r["bias"])
    out["rt_x"] = arr(r["in"])
    out["rt_idx"] = arr(r["topk_idx"], np.int32)
    out["rt_wt"] = arr(r["topk_weight"])
    out["rt_topk"] = np.int32(r["top_k"])
    out["rt_changed"] = np.int32(r["rows_where_bias_changed_selection"])
    s = json.load(open(os.path.join(REF, "ops", "situ_glu.json")))
    out["situ_in"] = arr(s["in"])
    out["situ_out"] = arr(s["out"])
    out["situ_b1"] = np.float32(s["beta"])
    out["situ_b2"] = np.float32(s["linear_beta"])
    n = json.load(open(os.path.join(REF, "ops", "rmsnorm.json")))
    out["rms_w"] = arr(n["weight"])
    out["rms_in"] = arr(n["in"])
    out["rms_out"] = arr(n["out"])
    out["rms_eps"] = np.float32(n["eps"])
    mo = json.load(open(os.path.join(REF, "ops", "moe.json")))
    for k in ("hidden", "latent", "moe_inter", "n_experts", "top_k", "n_shared", "renorm",
              "latent_norm"):
        out["moe_" + k] = np.int32(mo[k])
    for k in ("routed_scale", "rms_eps", "situ_b1", "situ_b2"):
        out["moe_" + k] = np.float32(mo[k])
    for k, v in mo.items():
        if isinstance(v, dict) and "data" in v:
            out["moe_t_" + k] = arr(v)
    man = json.load(open(os.path.join(REF, "ops", "MANIFEST.json")))
    out["tol_abs"] = np.float32(man["tolerance"]["fp32_abs"])
    out["tol_rel"] = np.float32(man["tolerance"]["fp32_rel"])
    np.savez_compressed(os.path.join(OUT, "ref_fixtures.npz"), **out)
    print("ref_fixtures.npz:", len(out), "arrays")


def edge_cases():
    """(name, packed, scales, x, in, rows, group) cases of the MXFP4 GEMV edge behaviour."""
    cases = []
    rng = np.random.default_rng(12345)
    # Scale-byte regimes, one per case so each is judged against its own magnitude:
    # subnormal and tiny (0..4: 2^-127 scales give fp32 / bf16 subnormal weights), the NaN
    # byte 255 mixed with ordinary scales (its blocks contribute nothing), and large but
    # finite (the fp32 sum cannot overflow).
    rows, inn = 64, 512
    for name, choices in (("scales_tiny", [0, 1, 2, 3, 4]),
                          ("scales_nan_byte", [126, 127, 128, 255]),
                          ("scales_large", list(range(200, 237)))):
        pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
        sc = rng.choice(np.array(choices, np.uint8), rows * inn // 32)
        x = rng.standard_normal(inn).astype(np.float32)
        cases.append((name, pk, sc, x, inn, rows, 32))
    for rows, inn in ((37, 96), (5, 2048), (130, 224), (1, 32), (17, 7168)):
        pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
        sc = rng.integers(119, 128, rows * ((inn + 31) // 32), dtype=np.uint8)
        x = rng.standard_normal(inn).astype(np.float32)
        cases.append((f"ragged_{rows}x{inn}", pk, sc, x, inn, rows, 32))
    rows, inn = 33, 80              # partial last group of 32
    pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
    sc = rng.integers(119, 128, rows * 3, dtype=np.uint8)
    x = rng.standard_normal(inn).astype(np.float32)
    cases.append(("partial_group", pk, sc, x, inn, rows, 32))
    rows, inn = 20, 96               # group 16 (flat path, 16 | group)
    pk = rng.integers(0, 256, rows * inn // 2, dtype=np.uint8)
    sc = rng.integers(119, 128, rows * 6, dtype=np.uint8)
    x = rng.standard_normal(inn).astype(np.float32)
    cases.append(("group16", pk, sc, x, inn, rows, 16))
    return cases


def reference_goldens():
    ref = Ref()
    g = {}
    packed, scales, x = wl.gemv_inputs()
    g["gemv_y"] = ref.matmul_mxfp4(x, packed, scales, wl.HIDDEN, 2048)
    e0 = wl.expert(0)
    xe = wl.expert_input()
    g["expert_silu"] = ref.expert_ffn(xe, e0, wl.HIDDEN, wl.INTER, act=1, wt=0.125)
    g["expert_situ"] = ref.expert_ffn(xe, e0, wl.HIDDEN, wl.INTER, act=0, wt=0.125)
    W = wl.router_weights()
    X = wl.tokens(64)
    idx = np.empty((64, wl.TOPK), np.int32)
    wt = np.empty((64, wl.TOPK), np.float32)
    for t in range(64):
        idx[t], wt[t] = ref.router(X[t], W, None, wl.TOPK)
    g["router_idx"], g["router_wt"] = idx, wt
    T = 8
    bank = wl.lazy_bank(idx[:T])
    out, i8, w8 = ref.moe_routed(X[:T], W, None, bank, wl.HIDDEN, wl.INTER, wl.TOPK, act=1)
    assert np.array_equal(i8, idx[:T])
    g["moe8_out"] = out
    for name, pk, sc, xx, inn, rows, group in edge_cases():
        g["edge_" + name] = ref.matmul_mxfp4(xx, pk, sc, inn, rows, group)
    np.savez_compressed(os.path.join(OUT, "ref_golden.npz"), **g)
    print("ref_golden.npz:", ", ".join(f"{k}{list(v.shape)}" for k, v in g.items()))


if __name__ == "__main__":
    if not Ref.available():
        sys.exit("oracle/_ref is not built: run make -C oracle")
    convert_reference_fixtures()
    reference_goldens()
