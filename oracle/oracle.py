# SPDX-License-Identifier: Apache-2.0
"""ctypes bindings of the CPU checkers. TEST INFRASTRUCTURE ONLY.

    Oracle()   liboracle.so, the restatement in k3_oracle.c (orc_* symbols)
    Ref()      _ref/libk3ref.so + _ref/libk3ref_compose.so: the reference's own
               src/core/k3_ops.c, compiled, and the routed-MoE composition over it

Both expose the same Python methods, so a test can run one input through either and
compare. Only tests/, the smoke entry point and bench.py's CPU-baseline leg use this.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
P, I, F = C.c_void_p, C.c_int, C.c_float


class ExpertQ(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("p1", "s1", "p3", "s3", "p2", "s2")]


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


class _Checker:
    prefix = None

    def _fn(self, name, res, *args):
        f = getattr(self.lib, name)
        f.restype = res
        f.argtypes = list(args)
        return f

    def _bind_common(self):
        pre = self.prefix
        self._mx = self._fn(pre + "matmul_mxfp4", None, P, P, P, P, I, I, I)
        self._dq = self._fn(pre + "mxfp4_dequant", None, P, P, P, I, I, I)
        self._mm = self._fn(pre + "matmul", None, P, P, P, I, I)
        self._mmb = self._fn(pre + "matmul_bf16", None, P, P, P, I, I)
        self._rt = self._fn(pre + "router", None, P, P, P, P, P, I, I, I, I, F)
        self._situ = self._fn(pre + "situ_glu", None, P, P, I, F, F)
        self._rms = self._fn(pre + "rmsnorm", None, P, P, P, I, F)

    def matmul_mxfp4(self, x, packed, scales, inn, rows, group=32):
        y = np.empty(rows, np.float32)
        self._mx(_p(y), _p(_f32(x)), _p(_u8(packed)), _p(_u8(scales)), inn, rows, group)
        return y

    def mxfp4_dequant(self, packed, scales, rows, pcols, group=32):
        out = np.empty((rows, pcols * 2), np.float32)
        self._dq(_p(out), _p(_u8(packed)), _p(_u8(scales)), rows, pcols, group)
        return out

    def matmul(self, x, W):
        W = _f32(W)
        y = np.empty(W.shape[0], np.float32)
        self._mm(_p(y), _p(_f32(x)), _p(W), W.shape[1], W.shape[0])
        return y

    def matmul_bf16(self, x, Wb):
        Wb = np.ascontiguousarray(Wb, dtype=np.uint16)
        y = np.empty(Wb.shape[0], np.float32)
        self._mmb(_p(y), _p(_f32(x)), _p(Wb), Wb.shape[1], Wb.shape[0])
        return y

    def router(self, x, W, bias, topk, renorm=1, routed_scale=1.0):
        W = _f32(W)
        idx = np.empty(topk, np.int32)
        w = np.empty(topk, np.float32)
        self._rt(_p(idx), _p(w), _p(_f32(x)), _p(W), _p(None if bias is None else _f32(bias)),
                 W.shape[1], W.shape[0], topk, renorm, routed_scale)
        return idx, w

    def situ_glu(self, x, n, b1=4.0, b2=25.0):
        y = np.empty(n, np.float32)
        self._situ(_p(y), _p(_f32(x)), n, b1, b2)
        return y

    def rmsnorm(self, x, w, eps):
        x = _f32(x)
        y = np.empty_like(x)
        self._rms(_p(y), _p(x), _p(_f32(w)), x.size, eps)
        return y

    @staticmethod
    def bank_structs(bank):
        qs = (ExpertQ * len(bank))()
        for e, ex in enumerate(bank):
            if ex is not None:
                qs[e] = ExpertQ(*[a.ctypes.data for a in ex.t])
        return qs


class Oracle(_Checker):
    prefix = "orc_"

    def __init__(self):
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run make -C oracle")
        self.lib = C.CDLL(path)
        self._bind_common()
        self._ffn = self._fn("orc_expert_ffn", None, P, P, C.POINTER(ExpertQ), I, I, I, F, F, F)
        self._moe = self._fn("orc_moe_routed", None, P, P, P, P, I, P, P, P, I, I, I, I, I, F,
                             I, F, F)
        self._gather = self._fn("orc_gather", None, P, P, P, I, I, I)
        self._silu = self._fn("orc_silu_glu", None, P, P, I)
        self._fnv = self._fn("orc_fnv1a", C.c_uint64, P, C.c_size_t)
        self._fill_f = self._fn("orc_fill_f", None, P, C.c_size_t, C.c_uint)
        self._fill_b = self._fn("orc_fill_b", None, P, C.c_size_t, C.c_uint)
        self._fill_bf16 = self._fn("orc_fill_bf16", None, P, C.c_size_t, C.c_uint)
        self._threads = self._fn("orc_threads", I)
        self._latent = self._fn("orc_moe_latent", None, P, P, P, P, I)
        self._ffn_many = self._fn("orc_expert_ffn_many", None, P, P, I, C.POINTER(ExpertQ), I, I,
                                  I, F, F)

    def threads(self):
        return self._threads()

    def expert_ffn_many(self, X, ex, hidden, inter, act=1, b1=4.0, b2=25.0):
        """orc_expert_ffn (combine weight 1) for every row of X, expert-major."""
        X = _f32(X).reshape(-1, hidden)
        out = np.empty((X.shape[0], hidden), np.float32)
        q = ExpertQ(*[a.ctypes.data for a in ex.t])
        self._ffn_many(_p(out), _p(X), X.shape[0], C.byref(q), hidden, inter, act, b1, b2)
        return out

    def moe_outputs(self, X, idx, wt, bank, hidden, inter, act=1, b1=4.0, b2=25.0):
        """out[t] = 0 + sum_j wt[t][j] * expert_ffn(idx[t][j], x[t]), j ascending, in fp32
        (k3_moe's routed loop, k3_ops.c:628-642), the experts evaluated expert-major.
        bank[e]: the host expert e (needed for every e in idx)."""
        X = _f32(X).reshape(-1, hidden)
        T, K = idx.shape
        contrib = np.empty((T, K, hidden), np.float32)
        for e in np.unique(idx):
            ts, js = np.nonzero(idx == e)
            contrib[ts, js] = self.expert_ffn_many(X[ts], bank[int(e)], hidden, inter, act, b1, b2)
        out = np.zeros((T, hidden), np.float32)
        for j in range(K):
            out = out + wt[:, j:j + 1].astype(np.float32) * contrib[:, j]
        return out

    def expert_ffn(self, x, ex, hidden, inter, act=1, b1=4.0, b2=25.0, wt=1.0):
        out = np.empty(hidden, np.float32)
        q = ExpertQ(*[a.ctypes.data for a in ex.t])
        self._ffn(_p(out), _p(_f32(x)), C.byref(q), hidden, inter, act, b1, b2, wt)
        return out

    def moe_routed(self, x, router_w, bias, bank, hidden, inter, topk, renorm=1,
                   routed_scale=1.0, act=1, b1=4.0, b2=25.0):
        x = _f32(x).reshape(-1, hidden)
        T = x.shape[0]
        out = np.empty((T, hidden), np.float32)
        idx = np.empty((T, topk), np.int32)
        wt = np.empty((T, topk), np.float32)
        qs = self.bank_structs(bank)
        self._moe(_p(out), _p(idx), _p(wt), _p(x), T, _p(_f32(router_w)),
                  _p(None if bias is None else _f32(bias)), qs, hidden, inter, len(bank), topk,
                  renorm, routed_scale, act, b1, b2)
        return out, idx, wt

    def gather(self, idx, n_experts):
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        T, topk = idx.shape
        offsets = np.empty(n_experts + 1, np.int32)
        perm = np.empty(T * topk, np.int32)
        self._gather(_p(offsets), _p(perm), _p(idx), T, topk, n_experts)
        return offsets, perm

    def silu_glu(self, x, n):
        y = np.empty(n, np.float32)
        self._silu(_p(y), _p(_f32(x)), n)
        return y

    def fnv1a(self, v):
        v = _f32(v)
        return int(self._fnv(_p(v), v.size))

    def fill_f(self, n, seed):
        a = np.empty(n, np.float32)
        self._fill_f(_p(a), n, seed)
        return a

    def fill_b(self, n, seed):
        a = np.empty(n, np.uint8)
        self._fill_b(_p(a), n, seed)
        return a

    def fill_bf16(self, n, seed):
        a = np.empty(n, np.uint16)
        self._fill_bf16(_p(a), n, seed)
        return a

    def moe_latent(self, x, cfg, W):
        """cfg: dict of the LatentMoE shape; W: dict of fp32 arrays (fixture names)."""
        class Cfg(C.Structure):
            _fields_ = [(n, I) for n in ("hidden", "latent", "inter", "n_experts", "topk",
                                        "n_shared", "renorm", "latent_norm")] + \
                       [(n, F) for n in ("routed_scale", "rms_eps", "b1", "b2")]

        class Wt(C.Structure):
            _fields_ = [(n, P) for n in ("gate", "bias", "w1", "w3", "w2", "latent_norm", "down",
                                        "up", "sh1", "sh3", "sh2")]
        keep = {k: _f32(v) for k, v in W.items()}
        c = Cfg(*[int(cfg[k]) for k in ("hidden", "latent", "inter", "n_experts", "topk",
                                         "n_shared", "renorm", "latent_norm")],
                *[float(cfg[k]) for k in ("routed_scale", "rms_eps", "b1", "b2")])
        w = Wt(*[keep[k].ctypes.data if k in keep else None for k in
                 ("gate", "bias", "w1", "w3", "w2", "latent_norm", "down", "up", "sh1", "sh3",
                  "sh2")])
        x = _f32(x).reshape(-1, c.hidden)
        out = np.empty_like(x)
        self._latent(_p(out), _p(x), C.byref(w), C.byref(c), x.shape[0])
        return out


def q8_rows(rng, inn, out):
    """Random k3_matmul_q8 weights: each row a float32 scale then inn int8 values."""
    sc = (rng.random(out) * 0.02 + 0.001).astype(np.float32)
    q = rng.integers(-128, 128, (out, inn), dtype=np.int64).astype(np.int8)
    W = np.empty((out, 4 + inn), np.uint8)
    W[:, :4] = sc.view(np.uint8).reshape(out, 4)
    W[:, 4:] = q.view(np.uint8)
    return W, sc, q


def q8_exact(x, sc, q):
    """k3_matmul_q8 in exact arithmetic: (sum_i q[o][i] * x[i]) * scale[o], in fp64
    (every product and the sum of 7168 of them are exact in fp64 up to one rounding per
    addition of magnitudes far below 2^53 ulps of the result)."""
    return (q.astype(np.float64) @ np.asarray(x, np.float64)) * sc.astype(np.float64)


class Ref(_Checker):
    """The compiled reference. Available wherever oracle/_ref was built."""
    prefix = "k3_"

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libk3ref_compose.so"))

    def __init__(self):
        base = os.path.join(HERE, "_ref")
        self.lib = C.CDLL(os.path.join(base, "libk3ref.so"), mode=C.RTLD_LOCAL)
        self.comp = C.CDLL(os.path.join(base, "libk3ref_compose.so"))
        self._bind_common()
        self._ffn = self.comp.ref_expert_ffn
        self._ffn.restype = I
        self._ffn.argtypes = [P, P, C.POINTER(ExpertQ), I, I, I, F, F, F]
        self._moe = self.comp.ref_moe_routed
        self._moe.restype = I
        self._moe.argtypes = [P, P, P, P, I, P, P, P, I, I, I, I, I, F, I, F, F]

    def matmul_q8(self, x, Wq, inn, out):
        """k3_matmul_q8 (k3_ops.c:1221-1289): rows of [f32 scale][int8 x inn]."""
        fn = self.lib.k3_matmul_q8
        fn.restype = None
        fn.argtypes = [P, P, P, I, I]
        y = np.empty(out, np.float32)
        fn(_p(y), _p(_f32(x)), _p(_u8(Wq)), inn, out)
        return y

    def expert_ffn(self, x, ex, hidden, inter, act=1, b1=4.0, b2=25.0, wt=1.0):
        out = np.empty(hidden, np.float32)
        q = ExpertQ(*[a.ctypes.data for a in ex.t])
        assert self._ffn(_p(out), _p(_f32(x)), C.byref(q), hidden, inter, act, b1, b2, wt) == 0
        return out

    def moe_routed(self, x, router_w, bias, bank, hidden, inter, topk, renorm=1,
                   routed_scale=1.0, act=1, b1=4.0, b2=25.0):
        x = _f32(x).reshape(-1, hidden)
        T = x.shape[0]
        out = np.empty((T, hidden), np.float32)
        idx = np.empty((T, topk), np.int32)
        wt = np.empty((T, topk), np.float32)
        qs = self.bank_structs(bank)
        assert self._moe(_p(out), _p(idx), _p(wt), _p(x), T, _p(_f32(router_w)),
                         _p(None if bias is None else _f32(bias)), qs, hidden, inter, len(bank),
                         topk, renorm, routed_scale, act, b1, b2) == 0
        return out, idx, wt


# ------------------------------------------------------- streamed-expert LatentMoE ----
class ExpertSrc(C.Structure):
    """The reference's K3ExpertSrc (include/k3/k3.h:332-355); the library under test declares
    the same layout, so one instance can be handed to the oracle, the compiled reference and
    the library."""


GETFN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.POINTER(ExpertQ))
GETMANYFN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.POINTER(C.c_int), C.c_int)
ExpertSrc._fields_ = [("get", GETFN), ("getmany", GETMANYFN), ("resident", GETFN),
                      ("ctx", C.c_void_p)]


class PySource:
    """A K3ExpertSrc over host experts. bank: {expert id: object with .t = the six arrays
    p1, s1, p3, s3, p2, s2}. get() fails for ids in `fail` (and for ids absent from the
    bank); resident() answers from `resident` (default: the whole bank). Every call is
    logged in .calls as (name, args)."""

    def __init__(self, bank, fail=(), resident=None, with_getmany=True, with_resident=True):
        self.bank = bank
        self.fail = set(fail)
        self.res = set(bank) if resident is None else set(resident)
        self.calls = []
        self._get = GETFN(self._cb_get)
        self._many = GETMANYFN(self._cb_getmany) if with_getmany else GETMANYFN()
        self._resf = GETFN(self._cb_resident) if with_resident else GETFN()
        self.struct = ExpertSrc(self._get, self._many, self._resf, None)

    def _fill(self, e, out):
        if out:
            out[0] = ExpertQ(*[a.ctypes.data for a in self.bank[e].t])

    def _cb_get(self, _self, layer, e, out):
        self.calls.append(("get", layer, e))
        if e in self.fail or e not in self.bank:
            return -1
        self._fill(e, out)
        return 0

    def _cb_getmany(self, _self, layer, experts, n):
        self.calls.append(("getmany", layer, tuple(experts[i] for i in range(n))))
        return sum(1 for i in range(n) if experts[i] in self.bank and experts[i] not in self.fail)

    def _cb_resident(self, _self, layer, e, out):
        self.calls.append(("resident", layer, e))
        if e not in self.res or e not in self.bank:
            return 0
        self._fill(e, out)
        return 1

    @property
    def ptr(self):
        return C.addressof(self.struct)


class RefCfg(C.Structure):
    """The reference's K3Cfg (include/k3/k3.h:73-120)."""
    _fields_ = [("hidden", I), ("n_layers", I), ("vocab", I), ("rms_eps", F),
                ("kda_heads", I), ("kda_head_dim", I), ("conv_k", I), ("gate_lb", F),
                ("n_heads", I), ("q_lora", I), ("kv_lora", I), ("qk_nope", I), ("qk_rope", I),
                ("v_head", I), ("mla_out_gate", I), ("n_experts", I), ("topk", I),
                ("n_shared", I), ("latent", I), ("moe_inter", I), ("routed_scale", F),
                ("moe_renorm", I), ("latent_norm", I), ("first_dense", I), ("dense_inter", I),
                ("attn_res_block", I), ("situ_b1", F), ("situ_b2", F), ("n_full_attn", I),
                ("full_attn", C.c_void_p)]


class RefMoeW(C.Structure):
    """The reference's K3MoeW (include/k3/k3.h:357-380)."""
    _fields_ = [("gate", P), ("bias", P), ("w1", P), ("w3", P), ("w2", P), ("latent_norm", P),
                ("down", P), ("up", P), ("sh1", P), ("sh3", P), ("sh2", P), ("wdt", I),
                ("src", P), ("layer", I), ("cache_only", I)]


class _OrcMoeCfg(C.Structure):
    _fields_ = [(n, I) for n in ("hidden", "latent", "inter", "n_experts", "topk", "n_shared",
                                "renorm", "latent_norm")] + \
               [(n, F) for n in ("routed_scale", "rms_eps", "b1", "b2")]


class _OrcMoeQW(C.Structure):
    _fields_ = [("gate", P), ("bias", P), ("latent_norm", P), ("down", P), ("up", P),
                ("sh1", P), ("sh3", P), ("sh2", P), ("wdt", I), ("src", P), ("layer", I),
                ("cache_only", I)]


def ref_cfg(cfg):
    """RefCfg from a dict with hidden, latent, inter, n_experts, topk, n_shared, renorm,
    latent_norm, routed_scale, rms_eps, b1, b2."""
    c = RefCfg()
    c.hidden, c.latent, c.moe_inter = cfg["hidden"], cfg["latent"], cfg["inter"]
    c.n_experts, c.topk, c.n_shared = cfg["n_experts"], cfg["topk"], cfg["n_shared"]
    c.moe_renorm, c.latent_norm = cfg["renorm"], cfg["latent_norm"]
    c.routed_scale, c.rms_eps = cfg["routed_scale"], cfg["rms_eps"]
    c.situ_b1, c.situ_b2 = cfg["b1"], cfg["b2"]
    return c


def ref_moew(W, wdt, src, layer=0, cache_only=0):
    """RefMoeW over a dict of arrays named gate, bias, latent_norm, down, up, sh1, sh3, sh2."""
    g = lambda k: W[k].ctypes.data if W.get(k) is not None else None  # noqa: E731
    return RefMoeW(g("gate"), g("bias"), None, None, None, g("latent_norm"), g("down"), g("up"),
                   g("sh1"), g("sh3"), g("sh2"), wdt, src.ptr if src is not None else None,
                   layer, cache_only)


def _bind_moe_q(obj):
    f = obj.lib.orc_moe_q
    f.restype = None
    f.argtypes = [P, P, P, P, I, P, P, I, C.POINTER(C.c_long)]
    return f


def oracle_moe_q(orc, x, cfg, W, wdt, src, prefill, layer=0, cache_only=0, idx=None, wt=None):
    """orc_moe_q: the streamed LatentMoE of the oracle. Returns out, idx, wt, drops (idx/wt
    start as the given arrays, or -7 / nan, so that untouched entries are visible)."""
    if not hasattr(orc, "_moe_q"):
        orc._moe_q = _bind_moe_q(orc)
    x = _f32(x).reshape(-1, cfg["hidden"])
    T = x.shape[0]
    c = _OrcMoeCfg(*[int(cfg[k]) for k in ("hidden", "latent", "inter", "n_experts", "topk",
                                            "n_shared", "renorm", "latent_norm")],
                   *[float(cfg[k]) for k in ("routed_scale", "rms_eps", "b1", "b2")])
    g = lambda k: W[k].ctypes.data if W.get(k) is not None else None  # noqa: E731
    w = _OrcMoeQW(g("gate"), g("bias"), g("latent_norm"), g("down"), g("up"), g("sh1"), g("sh3"),
                  g("sh2"), wdt, src.ptr, layer, cache_only)
    out = np.empty_like(x)
    K = cfg["topk"]
    idx = np.full(K, -7, np.int32) if idx is None else np.array(idx, np.int32)
    wt = np.full(K, np.nan, np.float32) if wt is None else np.array(wt, np.float32)
    drops = C.c_long(0)
    orc._moe_q(_p(out), _p(x), C.byref(w), C.byref(c), T, _p(idx), _p(wt), prefill,
               C.byref(drops))
    return out, idx, wt, drops.value


def ref_moe_q(ref, x, cfg, W, wdt, src, prefill, layer=0, cache_only=0, idx=None, wt=None):
    """The compiled reference's own k3_moe / k3_moe_prefill on the same inputs."""
    L = ref.lib
    fn = L.k3_moe_prefill if prefill else L.k3_moe
    fn.restype = None
    fn.argtypes = [P, P, C.POINTER(RefMoeW), C.POINTER(RefCfg), I, P, P, P]
    L.k3_moe_scratch.restype = C.c_size_t
    L.k3_moe_scratch.argtypes = [C.POINTER(RefCfg)]
    c = ref_cfg(cfg)
    w = ref_moew(W, wdt, src, layer, cache_only)
    x = _f32(x).reshape(-1, cfg["hidden"])
    out = np.empty_like(x)
    K = cfg["topk"]
    idx = np.full(K, -7, np.int32) if idx is None else np.array(idx, np.int32)
    wt = np.full(K, np.nan, np.float32) if wt is None else np.array(wt, np.float32)
    scratch = np.empty(L.k3_moe_scratch(C.byref(c)), np.float32)
    drops = C.c_long.in_dll(L, "k3_expert_drops")
    d0 = drops.value
    fn(_p(out), _p(x), C.byref(w), C.byref(c), x.shape[0], _p(idx), _p(wt), _p(scratch))
    return out, idx, wt, drops.value - d0
