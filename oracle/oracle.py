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

    def threads(self):
        return self._threads()

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


class Ref(_Checker):
    """The compiled reference. Available wherever oracle/_ref was built."""
    prefix = "k3_"

    @staticmethod
    def available():
        return os.path.exists(os.path.join(HERE, "_ref", "libk3ref_compose.so"))

    def __init__(self):
        base = os.path.join(HERE, "_ref")
        self.lib = C.CDLL(os.path.join(base, "libk3ref.so"), mode=C.RTLD_GLOBAL)
        self.comp = C.CDLL(os.path.join(base, "libk3ref_compose.so"))
        self._bind_common()
        self._ffn = self.comp.ref_expert_ffn
        self._ffn.restype = I
        self._ffn.argtypes = [P, P, C.POINTER(ExpertQ), I, I, I, F, F, F]
        self._moe = self.comp.ref_moe_routed
        self._moe.restype = I
        self._moe.argtypes = [P, P, P, P, I, P, P, P, I, I, I, I, I, F, I, F, F]

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
