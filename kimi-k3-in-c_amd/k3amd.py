# SPDX-License-Identifier: Apache-2.0
"""Python mirror of libk3amd.so's C ABI (include/k3.h, include/k3_dev.h, include/k3_gen.h).

The host-pointer functions keep the reference's names, argument meaning and error
behaviour (src/core/k3_ops.c of the reference; a precondition violation aborts the
process there and here). Arrays are numpy; outputs are returned. The device-pointer
functions take integer device addresses (e.g. torch tensor .data_ptr()) and a stream
handle, and enqueue without synchronising.

The library is loaded from this directory; nothing here falls back to another
implementation: if libk3amd.so is missing the import of any entry point raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libk3amd.so")

K3_WF32, K3_WBF16, K3_WI8 = 0, 1, 2
K3_ACT_SITU, K3_ACT_SILU = 0, 1
K3_MAX_TOPK = 64
K3D_LAYOUT_ROWS, K3D_LAYOUT_TILED = 0, 1
STAGES = ("begin", "router", "gather", "gateup", "down", "combine", "gemv", "shared")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        _lib = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
        _declare(_lib)
    return _lib


P = C.c_void_p
I = C.c_int
F = C.c_float
SZ = C.c_size_t


class K3ExpertQ(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("p1", "s1", "p3", "s3", "p2", "s2")]


class K3ExpertSrc(C.Structure):
    pass


GETFN = C.CFUNCTYPE(C.c_int, C.POINTER(K3ExpertSrc), C.c_int, C.c_int, C.POINTER(K3ExpertQ))
GETMANYFN = C.CFUNCTYPE(C.c_int, C.POINTER(K3ExpertSrc), C.c_int, C.POINTER(C.c_int), C.c_int)
K3ExpertSrc._fields_ = [("get", GETFN), ("getmany", GETMANYFN), ("resident", GETFN),
                        ("ctx", C.c_void_p)]


class K3Cfg(C.Structure):
    _fields_ = [("hidden", I), ("n_layers", I), ("vocab", I), ("rms_eps", F),
                ("kda_heads", I), ("kda_head_dim", I), ("conv_k", I), ("gate_lb", F),
                ("n_heads", I), ("q_lora", I), ("kv_lora", I), ("qk_nope", I), ("qk_rope", I),
                ("v_head", I), ("mla_out_gate", I), ("n_experts", I), ("topk", I),
                ("n_shared", I), ("latent", I), ("moe_inter", I), ("routed_scale", F),
                ("moe_renorm", I), ("latent_norm", I), ("first_dense", I), ("dense_inter", I),
                ("attn_res_block", I), ("situ_b1", F), ("situ_b2", F), ("n_full_attn", I),
                ("full_attn", C.POINTER(C.c_int))]


class K3MoeW(C.Structure):
    _fields_ = [("gate", P), ("bias", P), ("w1", P), ("w3", P), ("w2", P), ("latent_norm", P),
                ("down", P), ("up", P), ("sh1", P), ("sh3", P), ("sh2", P), ("wdt", I),
                ("src", P), ("layer", I), ("cache_only", I)]


class K3DevBankStats(C.Structure):
    _fields_ = [("hits", C.c_long), ("misses", C.c_long), ("evictions", C.c_long),
                ("failures", C.c_long), ("bytes_uploaded", C.c_ulonglong), ("resident", I),
                ("slots", I), ("slot_bytes", SZ)]


def _declare(L):
    def d(name, res, *args):
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = list(args)

    d("k3_matmul", None, P, P, P, I, I)
    d("k3_matmul_bf16", None, P, P, P, I, I)
    d("k3_matmul_q8", None, P, P, P, I, I)
    d("k3_mxfp4_dequant", None, P, P, P, I, I, I)
    d("k3_matmul_mxfp4", None, P, P, P, P, I, I, I)
    d("k3_router", None, P, P, P, P, P, I, I, I, I, F)
    d("k3_situ_glu", None, P, P, I, F, F)
    d("k3_rmsnorm", None, P, P, P, I, F)
    d("k3_moe_scratch", SZ, C.POINTER(K3Cfg))
    d("k3_moe", None, P, P, C.POINTER(K3MoeW), C.POINTER(K3Cfg), I, P, P, P)
    d("k3_moe_prefill", None, P, P, C.POINTER(K3MoeW), C.POINTER(K3Cfg), I, P, P, P)
    d("k3_expert_ffn", None, P, P, C.POINTER(K3ExpertQ), I, I, I, F, F, F)
    d("k3_moe_routed", None, P, P, P, P, I, P, P, P, I, I, I, I, I, F, I, F, F, I)
    d("k3_dev_register", I, P, SZ)
    d("k3_dev_unregister", I, P)
    d("k3_dev_lookup", P, P)
    d("k3_dev_last_error", C.c_char_p)
    d("k3_devbank_create", P, I, I, I, I, I, I, P)
    d("k3_devbank_source", P, P)
    d("k3_devbank_run_bytes", SZ, I, I)
    d("k3_devbank_put_run", I, P, I, I, P, SZ)
    d("k3_devbank_stats", I, P, C.POINTER(K3DevBankStats))
    d("k3_devbank_destroy", None, P)
    # device API
    d("k3d_init", I)
    d("k3d_error", C.c_char_p)
    d("k3d_malloc", P, SZ)
    d("k3d_free", I, P)
    d("k3d_h2d", I, P, P, SZ, P)
    d("k3d_d2h", I, P, P, SZ, P)
    d("k3d_sync", I, P)
    d("k3d_stream_create", P)
    d("k3d_stream_destroy", I, P)
    d("k3d_graph_begin", I, P)
    d("k3d_graph_end", I, P, P)
    d("k3d_graph_launch", I, P, P)
    d("k3d_graph_destroy", I, P)
    d("k3d_stamps_begin", I, P, SZ)
    d("k3d_stamps_end", I, P, P, I, P)
    d("k3d_prof_begin", I, I)
    d("k3d_prof_mark", I, P, I)
    d("k3d_prof_end", I, P, P, I)
    d("k3d_matmul_mxfp4_ws", SZ, I, I)
    d("k3d_matmul_mxfp4", I, P, P, I, P, P, I, I, I, P, SZ, P)
    d("k3d_matmul_f32", I, P, P, I, P, I, I, P)
    d("k3d_matmul_bf16", I, P, P, I, P, I, I, P)
    d("k3d_router_ws", SZ, I, I, I)
    d("k3d_router", I, P, P, P, I, P, P, I, I, I, I, F, P, SZ, P)
    d("k3d_router_recomputed", I, P, P, I, I, I)
    d("k3d_router_partials", I, P, P, P, SZ, P, I, I, I)
    d("k3d_moe_ws", SZ, I, I, I, I, I, I)
    d("k3d_moe_routed", I, P, P, P, P, I, P, P, P, I, I, I, I, I, I, F, I, F, F, I, P, SZ, P, P,
      P, P)
    d("k3d_static_ws_bytes", SZ)
    d("k3d_moe_routed_static", I, P, P, P, P, I, P, P, P, I, I, I, I, I, I, F, I, F, F, I, P, P, P,
      P)
    d("k3d_moe_experts", I, P, P, P, P, I, P, I, I, I, I, I, I, F, F, I, P, SZ, P, P, P, P)
    d("k3d_shared_ws", SZ, I, I, I, I)
    d("k3d_shared_expert", I, P, I, P, I, P, P, P, I, I, I, F, F, I, P, SZ, P)
    d("k3d_mxfp4_tiled_size", I, I, I, P, P)
    d("k3d_mxfp4_tile", I, P, P, P, P, I, I, P)
    # generator
    d("k3g_u64", C.c_uint64, C.c_uint64, C.c_uint64)
    d("k3g_bytes", None, P, SZ, C.c_uint64)
    d("k3g_e8m0", None, P, SZ, C.c_uint64, I, I)
    d("k3g_normal", None, P, SZ, C.c_uint64, C.c_double, C.c_double)
    d("k3g_bf16_normal", None, P, SZ, C.c_uint64, C.c_double, C.c_double)
    d("k3g_expert_seed", C.c_uint64, C.c_uint64, I, I)
    d("k3g_mxfp4_expert", None, P, P, P, P, P, P, I, I, C.c_uint64, I, I, I)


def exported_symbols():
    """Names this module binds; the C-ABI tests check the library exports each one."""
    return ["k3_matmul", "k3_matmul_bf16", "k3_matmul_q8", "k3_mxfp4_dequant",
            "k3_matmul_mxfp4", "k3_router", "k3_situ_glu", "k3_rmsnorm", "k3_moe_scratch",
            "k3_moe", "k3_moe_prefill", "k3_expert_ffn", "k3_moe_routed", "k3_dev_register",
            "k3_dev_unregister", "k3_dev_lookup", "k3_dev_last_error", "k3_expert_drops",
            "k3_devbank_create", "k3_devbank_source", "k3_devbank_run_bytes",
            "k3_devbank_put_run", "k3_devbank_stats", "k3_devbank_destroy"]


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


# ------------------------------------------------------------------ host surface ----
def matmul(x, W):
    W = _f32(W)
    out, inn = W.shape
    y = np.empty(out, np.float32)
    lib().k3_matmul(_p(y), _p(_f32(x)), _p(W), inn, out)
    return y


def matmul_bf16(x, Wb):
    Wb = np.ascontiguousarray(Wb, dtype=np.uint16)
    out, inn = Wb.shape
    y = np.empty(out, np.float32)
    lib().k3_matmul_bf16(_p(y), _p(_f32(x)), _p(Wb), inn, out)
    return y


def matmul_q8(x, Wq, inn, out):
    Wq = _u8(Wq)
    y = np.empty(out, np.float32)
    lib().k3_matmul_q8(_p(y), _p(_f32(x)), _p(Wq), inn, out)
    return y


def matmul_mxfp4(x, packed, scales, inn, rows, group=32):
    y = np.empty(rows, np.float32)
    lib().k3_matmul_mxfp4(_p(y), _p(_f32(x)), _p(_u8(packed)), _p(_u8(scales)), inn, rows, group)
    return y


def mxfp4_dequant(packed, scales, rows, pcols, group=32):
    out = np.empty((rows, pcols * 2), np.float32)
    lib().k3_mxfp4_dequant(_p(out), _p(_u8(packed)), _p(_u8(scales)), rows, pcols, group)
    return out


def router(x, W, bias, topk, renorm=1, routed_scale=1.0):
    W = _f32(W)
    n_experts, hidden = W.shape
    idx = np.empty(topk, np.int32)
    w = np.empty(topk, np.float32)
    b = None if bias is None else _f32(bias)
    lib().k3_router(_p(idx), _p(w), _p(_f32(x)), _p(W), _p(b), hidden, n_experts, topk, renorm,
                    routed_scale)
    return idx, w


def situ_glu(x, n, b1=4.0, b2=25.0):
    y = np.empty(n, np.float32)
    lib().k3_situ_glu(_p(y), _p(_f32(x)), n, b1, b2)
    return y


def rmsnorm(x, w, eps):
    x = _f32(x)
    y = np.empty_like(x)
    lib().k3_rmsnorm(_p(y), _p(x), _p(_f32(w)), x.size, eps)
    return y


class Expert:
    """One MXFP4 expert held in host memory (gate/up [inter][hidden], down [hidden][inter])."""

    def __init__(self, p1, s1, p3, s3, p2, s2):
        self.t = [_u8(a) for a in (p1, s1, p3, s3, p2, s2)]

    def q(self):
        return K3ExpertQ(*[a.ctypes.data for a in self.t])


def gen_expert(hidden, inter, seed, expert, lo=119, hi=127):
    pk = hidden * inter // 2
    sc = hidden * inter // 32
    a = [np.empty(n, np.uint8) for n in (pk, sc, pk, sc, pk, sc)]
    lib().k3g_mxfp4_expert(*[_p(t) for t in a], hidden, inter, seed, expert, lo, hi)
    return Expert(*a)


def expert_ffn(x, e, hidden, inter, act=K3_ACT_SILU, b1=4.0, b2=25.0, wt=1.0):
    out = np.empty(hidden, np.float32)
    q = e.q()
    lib().k3_expert_ffn(_p(out), _p(_f32(x)), C.byref(q), hidden, inter, act, b1, b2, wt)
    return out


def moe_routed(x, router_w, bias, bank, hidden, inter, topk, renorm=1, routed_scale=1.0,
               act=K3_ACT_SILU, b1=4.0, b2=25.0, prec=0):
    """bank: list of Expert (or None for a missing expert), one per expert id."""
    x = _f32(x).reshape(-1, hidden)
    T = x.shape[0]
    n_experts = len(bank)
    qs = (K3ExpertQ * n_experts)()
    for e, ex in enumerate(bank):
        if ex is not None:
            qs[e] = ex.q()
    out = np.empty((T, hidden), np.float32)
    idx = np.empty((T, topk), np.int32)
    wt = np.empty((T, topk), np.float32)
    b = None if bias is None else _f32(bias)
    lib().k3_moe_routed(_p(out), _p(idx), _p(wt), _p(x), T, _p(_f32(router_w)), _p(b), qs, hidden,
                        inter, n_experts, topk, renorm, routed_scale, act, b1, b2, prec)
    return out, idx, wt


def expert_drops():
    return C.c_long.in_dll(lib(), "k3_expert_drops").value


def cfg_struct(cfg):
    """K3Cfg from a dict with hidden, latent, inter, n_experts, topk, n_shared, renorm,
    latent_norm, routed_scale, rms_eps, b1, b2 (the MoE fields; the rest stay zero)."""
    c = K3Cfg()
    c.hidden, c.latent, c.moe_inter = cfg["hidden"], cfg["latent"], cfg["inter"]
    c.n_experts, c.topk, c.n_shared = cfg["n_experts"], cfg["topk"], cfg["n_shared"]
    c.moe_renorm, c.latent_norm = cfg["renorm"], cfg["latent_norm"]
    c.routed_scale, c.rms_eps = cfg["routed_scale"], cfg["rms_eps"]
    c.situ_b1, c.situ_b2 = cfg["b1"], cfg["b2"]
    return c


def moe(x, cfg, W, wdt, src_ptr, prefill, layer=0, cache_only=0, idx=None, wt=None):
    """k3_moe (prefill 0) or k3_moe_prefill (prefill 1) through the library. W: dict of
    host arrays gate, bias, latent_norm, down, up, sh1, sh3, sh2 (w1/w3/w2 for the
    resident fp32 bank); src_ptr: address of a K3ExpertSrc or None. Returns out, idx, wt
    (the topk-wide buffers after the call, initialised to -7 / nan unless given) and the
    increase of k3_expert_drops."""
    c = cfg_struct(cfg)
    g = lambda k: W[k].ctypes.data if W.get(k) is not None else None  # noqa: E731
    w = K3MoeW(g("gate"), g("bias"), g("w1"), g("w3"), g("w2"), g("latent_norm"), g("down"),
               g("up"), g("sh1"), g("sh3"), g("sh2"), wdt, src_ptr, layer, cache_only)
    x = _f32(x).reshape(-1, cfg["hidden"])
    out = np.empty_like(x)
    K = cfg["topk"]
    idx = np.full(K, -7, np.int32) if idx is None else np.array(idx, np.int32)
    wt = np.full(K, np.nan, np.float32) if wt is None else np.array(wt, np.float32)
    scratch = np.empty(lib().k3_moe_scratch(C.byref(c)), np.float32)
    d0 = expert_drops()
    fn = lib().k3_moe_prefill if prefill else lib().k3_moe
    fn(_p(out), _p(x), C.byref(w), C.byref(c), x.shape[0], _p(idx), _p(wt), _p(scratch))
    return out, idx, wt, expert_drops() - d0


class HbmBank:
    """k3_devbank_*: an expert bank in HBM behind a K3ExpertSrc."""

    def __init__(self, n_layers, n_experts, width, inter, slots, layout=K3D_LAYOUT_TILED,
                 upstream_ptr=None):
        self.h = lib().k3_devbank_create(n_layers, n_experts, width, inter, slots, layout,
                                         upstream_ptr)
        if not self.h:
            raise RuntimeError("k3_devbank_create: " + lib().k3_dev_last_error().decode())
        self.src = lib().k3_devbank_source(self.h)
        self.width, self.inter = width, inter

    def put_run(self, layer, expert, run):
        run = _u8(run)
        rc = lib().k3_devbank_put_run(self.h, layer, expert, run.ctypes.data, run.nbytes)
        if rc != 0:
            raise RuntimeError("k3_devbank_put_run: " + lib().k3_dev_last_error().decode())

    def stats(self):
        st = K3DevBankStats()
        check_dev(lib().k3_devbank_stats(self.h, C.byref(st)), "k3_devbank_stats")
        return {k: getattr(st, k) for k, _ in K3DevBankStats._fields_}

    def destroy(self):
        if self.h:
            lib().k3_devbank_destroy(self.h)
            self.h = None


def check_dev(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().k3_dev_last_error().decode()}")


def dev_register(arr):
    rc = lib().k3_dev_register(arr.ctypes.data, arr.nbytes)
    if rc != 0:
        raise RuntimeError(lib().k3_dev_last_error().decode())


def dev_unregister(arr):
    return lib().k3_dev_unregister(arr.ctypes.data)


# --------------------------------------------------------------------- generator ----
def gen_bytes(n, seed):
    a = np.empty(n, np.uint8)
    lib().k3g_bytes(_p(a), n, seed)
    return a


def gen_e8m0(n, seed, lo=119, hi=127):
    a = np.empty(n, np.uint8)
    lib().k3g_e8m0(_p(a), n, seed, lo, hi)
    return a


def gen_normal(n, seed, mean=0.0, sigma=1.0):
    a = np.empty(n, np.float32)
    lib().k3g_normal(_p(a), n, seed, mean, sigma)
    return a


def gen_bf16_normal(n, seed, mean=0.0, sigma=1.0):
    a = np.empty(n, np.uint16)
    lib().k3g_bf16_normal(_p(a), n, seed, mean, sigma)
    return a


def expert_seed(seed, expert, tensor):
    return lib().k3g_expert_seed(seed, expert, tensor)


# ------------------------------------------------------------------ device API ----
def check(rc, what="k3d"):
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().k3d_error().decode()}")


class Profile:
    """HIP-event stage timing of the library's own launches (k3d_prof_*)."""

    def __init__(self, max_marks=65536):
        check(lib().k3d_prof_begin(max_marks), "k3d_prof_begin")

    def end(self):
        n = len(STAGES)
        ms = (C.c_double * n)()
        cnt = (C.c_int * n)()
        check(lib().k3d_prof_end(ms, cnt, n), "k3d_prof_end")
        return {STAGES[i]: (ms[i], cnt[i]) for i in range(n) if cnt[i]}


class DevBuf:
    """A device allocation owned by Python (k3d_malloc / k3d_free)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().k3d_malloc(self.nbytes)
        if not self.ptr:
            raise RuntimeError("k3d_malloc: " + lib().k3d_error().decode())

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        check(lib().k3d_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, None), "h2d")
        check(lib().k3d_sync(None), "sync")
        return self

    def download(self, arr, offset=0):
        check(lib().k3d_d2h(arr.ctypes.data, self.ptr + offset, arr.nbytes, None), "d2h")
        check(lib().k3d_sync(None), "sync")
        return arr

    def free(self):
        if self.ptr:
            lib().k3d_free(self.ptr)
            self.ptr = None


class DevBank:
    """An expert bank resident on the device: the n experts' six MXFP4 arrays in HBM and a
    device table of K3ExpertQ with device pointers (None in `experts` = a dropped expert,
    NULL pointers in the table). layout K3D_LAYOUT_TILED stores each matrix regrouped by
    k3d_mxfp4_tile (the arrays are uploaded row-major into a staging buffer and tiled on the
    device); K3D_LAYOUT_ROWS stores them as they are."""

    def __init__(self, experts, hidden, inter, layout=K3D_LAYOUT_ROWS):
        L = lib()
        check(L.k3d_init(), "k3d_init")
        self.layout, self.n = layout, len(experts)
        shapes = [(inter, hidden), (inter, hidden), (hidden, inter)]   # (rows, in) of p1, p3, p2
        sizes = []
        for rows, inn in shapes:
            if layout == K3D_LAYOUT_TILED:
                pk, sc = C.c_size_t(), C.c_size_t()
                check(L.k3d_mxfp4_tiled_size(rows, inn, C.byref(pk), C.byref(sc)),
                      "k3d_mxfp4_tiled_size")
                sizes += [pk.value, sc.value]
            else:
                sizes += [rows * inn // 2, rows * inn // 32]
        rnd = [(b + 255) // 256 * 256 for b in sizes]
        slot = sum(rnd)
        self.mem = DevBuf(max(1, slot * self.n))
        stage = DevBuf(max(rnd)) if layout == K3D_LAYOUT_TILED else None
        stage2 = DevBuf(max(rnd)) if layout == K3D_LAYOUT_TILED else None
        table = (K3ExpertQ * max(1, self.n))()
        for e, ex in enumerate(experts):
            if ex is None:
                continue
            base = self.mem.ptr + e * slot
            offs = [base + sum(rnd[:i]) for i in range(6)]
            if layout == K3D_LAYOUT_TILED:
                for m, (rows, inn) in enumerate(shapes):
                    stage.upload(ex.t[2 * m])
                    stage2.upload(ex.t[2 * m + 1])
                    check(L.k3d_mxfp4_tile(offs[2 * m], offs[2 * m + 1], stage.ptr, stage2.ptr,
                                           rows, inn, None), "k3d_mxfp4_tile")
                    check(L.k3d_sync(None), "sync")
            else:
                for i in range(6):
                    self.mem.upload(ex.t[i], offs[i] - self.mem.ptr)
            table[e] = K3ExpertQ(*offs)
        for b in (stage, stage2):
            if b is not None:
                b.free()
        self.table = DevBuf(C.sizeof(table))
        check(L.k3d_h2d(self.table.ptr, C.addressof(table), C.sizeof(table), None), "h2d")
        check(L.k3d_sync(None), "sync")

    def free(self):
        self.mem.free()
        self.table.free()


def moe_routed_device(bank, x, router_w, bias, topk, renorm=1, routed_scale=1.0,
                      act=K3_ACT_SILU, b1=4.0, b2=25.0, prec=0, hidden=None, inter=None,
                      want_perm=True):
    """The routed layer through k3d_moe_routed on a DevBank: host arrays in, host arrays
    out (out [T][hidden], idx, wt [T][topk], perm [T*topk], offsets [n+1], drops). With
    want_perm False no permutation is asked for (perm and offsets come back None): a few
    tokens then take the path whose decode gate/up kernel selects the experts itself."""
    L = lib()
    router_w = _f32(router_w)
    n_experts, hid = router_w.shape
    hidden = hidden or hid
    x = _f32(x).reshape(-1, hidden)
    T = x.shape[0]
    bufs = {}
    try:
        bufs["x"] = DevBuf(x.nbytes).upload(x)
        bufs["w"] = DevBuf(router_w.nbytes).upload(router_w)
        bufs["b"] = DevBuf(n_experts * 4).upload(_f32(bias)) if bias is not None else None
        bufs["out"] = DevBuf(T * hidden * 4)
        bufs["idx"] = DevBuf(T * topk * 4)
        bufs["wt"] = DevBuf(T * topk * 4)
        bufs["perm"] = DevBuf(T * topk * 4) if want_perm else None
        bufs["off"] = DevBuf((n_experts + 1) * 4) if want_perm else None
        bufs["drops"] = DevBuf(4)
        wsb = L.k3d_moe_ws(T, hidden, inter, n_experts, topk, prec)
        bufs["ws"] = DevBuf(wsb)
        b = bufs["b"].ptr if bufs["b"] is not None else None
        check(L.k3d_moe_routed(bufs["out"].ptr, bufs["idx"].ptr, bufs["wt"].ptr, bufs["x"].ptr, T,
                               bufs["w"].ptr, b, bank.table.ptr, bank.layout, hidden, inter,
                               n_experts, topk, renorm, routed_scale, act, b1, b2, prec,
                               bufs["ws"].ptr, wsb, bufs["perm"].ptr if want_perm else None,
                               bufs["off"].ptr if want_perm else None,
                               bufs["drops"].ptr, None), "k3d_moe_routed")
        check(L.k3d_sync(None), "sync")
        out = bufs["out"].download(np.empty((T, hidden), np.float32))
        idx = bufs["idx"].download(np.empty((T, topk), np.int32))
        wt = bufs["wt"].download(np.empty((T, topk), np.float32))
        perm = bufs["perm"].download(np.empty(T * topk, np.int32)) if want_perm else None
        off = bufs["off"].download(np.empty(n_experts + 1, np.int32)) if want_perm else None
        drops = int(bufs["drops"].download(np.empty(1, np.int32))[0])
        return out, idx, wt, perm, off, drops
    finally:
        for v in bufs.values():
            if v is not None:
                v.free()


def moe_experts_device(bank, x, idx, wt, n_experts, act=K3_ACT_SILU, b1=4.0, b2=25.0, prec=0,
                       hidden=None, inter=None):
    """The expert half through k3d_moe_experts for a given routing (idx, wt [T][topk]) on a
    DevBank: host arrays in, (out [T][hidden], offsets [n+1], drops) out."""
    L = lib()
    x = _f32(x).reshape(-1, hidden)
    T = x.shape[0]
    idx = np.ascontiguousarray(idx, np.int32).reshape(T, -1)
    topk = idx.shape[1]
    wt = _f32(wt).reshape(T, topk)
    bufs = {}
    try:
        bufs["x"] = DevBuf(x.nbytes).upload(x)
        bufs["idx"] = DevBuf(idx.nbytes).upload(idx)
        bufs["wt"] = DevBuf(wt.nbytes).upload(wt)
        bufs["out"] = DevBuf(T * hidden * 4)
        bufs["perm"] = DevBuf(T * topk * 4)
        bufs["off"] = DevBuf((n_experts + 1) * 4)
        bufs["drops"] = DevBuf(4)
        wsb = L.k3d_moe_ws(T, hidden, inter, n_experts, topk, prec)
        bufs["ws"] = DevBuf(wsb)
        check(L.k3d_moe_experts(bufs["out"].ptr, bufs["idx"].ptr, bufs["wt"].ptr, bufs["x"].ptr, T,
                                bank.table.ptr, bank.layout, hidden, inter, n_experts, topk, act, b1,
                                b2, prec, bufs["ws"].ptr, wsb, bufs["perm"].ptr, bufs["off"].ptr,
                                bufs["drops"].ptr, None), "k3d_moe_experts")
        check(L.k3d_sync(None), "sync")
        out = bufs["out"].download(np.empty((T, hidden), np.float32))
        off = bufs["off"].download(np.empty(n_experts + 1, np.int32))
        drops = int(bufs["drops"].download(np.empty(1, np.int32))[0])
        return out, off, drops
    finally:
        for v in bufs.values():
            v.free()


def router_device(x, W, bias, topk, renorm=1, routed_scale=1.0, partials=False):
    """k3d_router over T tokens on the device: host arrays in, idx/wt [T][topk] out.
    partials: also fetch the chunk partials into router_device.partials = (part [ks][T][N],
    rbound [ks][T][N], chunk)."""
    L = lib()
    W = _f32(W)
    n_experts, hidden = W.shape
    x = _f32(x).reshape(-1, hidden)
    T = x.shape[0]
    bufs = [DevBuf(x.nbytes).upload(x), DevBuf(W.nbytes).upload(W),
            DevBuf(n_experts * 4).upload(_f32(bias)) if bias is not None else None,
            DevBuf(T * topk * 4), DevBuf(T * topk * 4)]
    wsb = L.k3d_router_ws(T, hidden, n_experts)
    bufs.append(DevBuf(wsb))
    try:
        dx, dW, db, di, dw, dws = bufs
        check(L.k3d_router(di.ptr, dw.ptr, dx.ptr, T, dW.ptr, db.ptr if db else None, hidden,
                           n_experts, topk, renorm, routed_scale, dws.ptr, wsb, None), "k3d_router")
        check(L.k3d_sync(None), "sync")
        rec = np.empty(T, np.int32)
        check(L.k3d_router_recomputed(rec.ctypes.data, dws.ptr, T, hidden, n_experts),
              "k3d_router_recomputed")
        router_device.recomputed = rec
        if partials:
            cap = ((hidden + 63) // 64) * T * n_experts
            part = np.empty(cap, np.float64)
            rb = np.empty(cap, np.float32)
            ch = np.zeros(1, np.int32)
            ks = L.k3d_router_partials(part.ctypes.data, rb.ctypes.data, ch.ctypes.data, cap, dws.ptr, T,
                                       hidden, n_experts)
            if ks <= 0:
                raise RuntimeError("k3d_router_partials: " + L.k3d_error().decode())
            n = ks * T * n_experts
            router_device.partials = (part[:n].reshape(ks, T, n_experts), rb[:n].reshape(ks, T, n_experts),
                                      int(ch[0]))
        return (di.download(np.empty((T, topk), np.int32)),
                dw.download(np.empty((T, topk), np.float32)))
    finally:
        for b in bufs:
            if b is not None:
                b.free()


def shared_expert_device(x, w1, w3, w2, hidden, inter, act=K3_ACT_SILU, b1=4.0, b2=25.0,
                         prec=0, y0=None):
    """k3d_shared_expert on host arrays: w1, w3 [inter][hidden], w2 [hidden][inter] as bf16
    bit patterns (uint16). Returns s (y0 None) or y0 + s."""
    L = lib()
    x = _f32(x).reshape(-1, hidden)
    T = x.shape[0]
    ws_b = L.k3d_shared_ws(T, hidden, inter, prec)
    bufs = [DevBuf(x.nbytes).upload(x), DevBuf(w1.nbytes).upload(w1), DevBuf(w3.nbytes).upload(w3),
            DevBuf(w2.nbytes).upload(w2), DevBuf(T * hidden * 4), DevBuf(ws_b)]
    try:
        dx, d1, d3, d2, dy, dws = bufs
        if y0 is not None:
            dy.upload(_f32(y0).reshape(T, hidden))
        check(L.k3d_shared_expert(dy.ptr, 1 if y0 is not None else 0, dx.ptr, T, d1.ptr, d3.ptr,
                                  d2.ptr, hidden, inter, act, b1, b2, prec, dws.ptr, ws_b, None),
              "k3d_shared_expert")
        check(L.k3d_sync(None), "sync")
        return dy.download(np.empty((T, hidden), np.float32))
    finally:
        for b in bufs:
            b.free()
