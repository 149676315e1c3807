# SPDX-License-Identifier: Apache-2.0
"""ctypes bindings for the CPU oracle (oracle/liboracle.so) and, where it
was built, the reference engine harness (oracle/_ref/libwasteref.so).

Test infrastructure: imported by tests/, the smoke check and bench.py's
cpu_baseline leg only.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libwasteref.so")

fp = C.POINTER(C.c_float)
u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
i8p = C.POINTER(C.c_int8)
i32p = C.POINTER(C.c_int)


def ptr(a, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


class OrcTensor(C.Structure):
    _fields_ = [("fmt", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("group", C.c_int),
                ("q", C.c_void_p), ("qs", u16p), ("rowbytes", C.c_size_t)]


class OrcRouteCfg(C.Structure):
    _fields_ = [("n_experts", C.c_int), ("top_k", C.c_int), ("score_func", C.c_int),
                ("renorm", C.c_int), ("routed_scale", C.c_float), ("n_group", C.c_int),
                ("topk_group", C.c_int)]


class OrcMoe(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
                ("moe_inter", C.c_int), ("n_shared", C.c_int), ("score_func", C.c_int),
                ("renorm", C.c_int), ("routed_scale", C.c_float), ("n_group", C.c_int),
                ("topk_group", C.c_int), ("stages", C.c_int), ("entries", C.c_int),
                ("vec_dim", C.c_int), ("order", C.c_int), ("router", OrcTensor),
                ("bias", fp), ("sh_gate", OrcTensor), ("sh_up", OrcTensor),
                ("sh_down", OrcTensor), ("booksT", fp), ("n_books", C.c_int),
                ("recs", C.POINTER(u8p)), ("rec_bytes", C.c_size_t)]


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


class Oracle:
    PORTABLE, AVX512 = 0, 1

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        _sig(L, "orc_expf", C.c_float, [C.c_float])
        _sig(L, "orc_f16_scale", C.c_float, [C.c_uint16])
        _sig(L, "orc_f16_book", C.c_float, [C.c_uint16])
        _sig(L, "orc_crc32", C.c_uint32, [u8p, C.c_size_t])
        _sig(L, "orc_books_load", None, [u16p, C.c_int, C.c_int, C.c_int, fp, fp])
        _sig(L, "orc_lutb", None, [fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "orc_vq_rows", None, [fp, u8p, u16p, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "orc_vq_quant_lut", None, [fp, C.c_int, C.c_int, C.c_int, i8p, fp])
        _sig(L, "orc_vq_rows_p6", None, [fp, u8p, u16p, i8p, fp, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "orc_dequant", None, [fp, u8p, u16p, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "orc_mvq_rows", None, [fp, i8p, u16p, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_size_t, C.c_int])
        _sig(L, "orc_matvec_f32", None, [fp, fp, fp, C.c_int, C.c_int])
        _sig(L, "orc_router_scores", None, [C.c_int, fp, fp, C.c_int])
        _sig(L, "orc_act_pair", None, [fp, fp, C.c_int])
        _sig(L, "orc_route", C.c_int, [C.POINTER(OrcRouteCfg), fp, fp, fp, i32p, fp])
        _sig(L, "orc_record_check", C.c_int, [u8p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "orc_moe_layer", C.c_int, [C.POINTER(OrcMoe), fp, fp, i32p, fp, fp])
        _sig(L, "orc_moe_chunk", C.c_int, [C.POINTER(OrcMoe), fp, C.c_int, fp, i32p, fp])
        _sig(L, "orc_moe_layer_mt", C.c_int, [C.POINTER(OrcMoe), fp, fp, i32p, fp, C.c_int])
        _sig(L, "orc_cpu_isa", C.c_int, [])
        _sig(L, "orc_moe_apply", C.c_int, [C.POINTER(OrcMoe), fp, C.c_int, i32p, fp, C.c_int, fp])
        _sig(L, "orc_router_logits", None, [C.POINTER(OrcMoe), fp, C.c_int, fp])
        _sig(L, "orc_ecache_new", C.c_void_p, [C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "orc_ecache_free", None, [C.c_void_p])
        for n in ("orc_ecache_hint", "orc_ecache_prefetch"):
            _sig(L, n, None, [C.c_void_p, C.c_int, i32p, C.c_int])
        for n in ("orc_ecache_get", "orc_ecache_hold", "orc_ecache_admit"):
            _sig(L, n, C.c_int, [C.c_void_p, C.c_int, C.c_int])
        _sig(L, "orc_ecache_release", None, [C.c_void_p])
        _sig(L, "orc_ecache_resident_mask", None, [C.c_void_p, C.c_int, C.c_int, u8p])
        _sig(L, "orc_ecache_stats", None, [C.c_void_p, C.POINTER(C.c_uint64)])
        _sig(L, "orc_predict_next", C.c_int, [C.c_int, C.c_int, fp, fp, C.c_int, i32p])

    def vq_quant_lut(self, lut, nv, stages=4, entries=64):
        """VQ4P's int8 table and per-32-position scales (src/model.c:3979-4074)."""
        lut = np.ascontiguousarray(lut, np.float32)
        q = np.zeros(nv * stages * entries, np.int8)
        sc = np.zeros((nv + 31) // 32, np.float32)
        self.lib.orc_vq_quant_lut(ptr(lut, fp), nv, stages, entries, ptr(q, i8p), ptr(sc, fp))
        return q, sc

    def vq_rows_p6(self, idx, scale, lut8, lscale, M, nv, order, r_lo=0):
        """VQ4P rows [r_lo, M) through the int8 table (src/model.c:4076-4114)."""
        idx = np.ascontiguousarray(idx, np.uint8)
        scale = np.ascontiguousarray(scale, np.uint16)
        lut8 = np.ascontiguousarray(lut8, np.int8)
        lscale = np.ascontiguousarray(lscale, np.float32)
        y = np.zeros(M, np.float32)
        self.lib.orc_vq_rows_p6(ptr(y, fp), ptr(idx, u8p), ptr(scale, u16p), ptr(lut8, i8p), ptr(lscale, fp),
                                r_lo, M, nv, order)
        return y

    def ecache_run(self, ops, n_slots, depth, policy, masks=None):
        """Runs a cache script (tests/ecache_script.py) through the
        restatement: (outputs, [hits, misses, evictions, prefetched,
        spec_issued, reads]).  masks: {word index: (layer, n)} to record
        resident_mask before that op."""
        L = self.lib
        c = L.orc_ecache_new(n_slots, depth if depth > 0 else 1, 1 if depth > 0 else 0, policy)
        out, got = [], {}
        w = 0
        while w < len(ops):
            if masks and w in masks:
                layer, n = masks[w]
                m = np.zeros(n, np.uint8)
                L.orc_ecache_resident_mask(c, layer, n, ptr(m, u8p))
                got[w] = m
            op = ops[w]
            if op in (0, 1, 5):
                f = (L.orc_ecache_get, L.orc_ecache_hold, None, None, None, L.orc_ecache_admit)[op]
                out.append(f(c, ops[w + 1], ops[w + 2]))
                w += 3
            elif op == 2:
                L.orc_ecache_release(c)
                w += 1
            else:
                n = ops[w + 2]
                a = np.array(ops[w + 3:w + 3 + n] or [0], np.int32)
                (L.orc_ecache_hint if op == 3 else L.orc_ecache_prefetch)(c, ops[w + 1], ptr(a, i32p), n)
                w += 3 + n
        st = (C.c_uint64 * 6)()
        L.orc_ecache_stats(c, st)
        L.orc_ecache_free(c)
        return (out, list(st), got) if masks else (out, list(st))

    def predict_next(self, score_func, logits, bias, n):
        lg = np.ascontiguousarray(logits, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        out = np.full(max(n, 1), -7, np.int32)
        k = self.lib.orc_predict_next(score_func, lg.size, ptr(lg, fp), ptr(b, fp), n, ptr(out, i32p))
        return out[:k]

    def expf(self, x):
        return self.lib.orc_expf(float(x))

    def books(self, books_f16):
        nb, en = books_f16.shape[0], books_f16.shape[1]
        b = np.zeros((nb, en, 8), np.float32)
        bt = np.zeros((nb, 8, en), np.float32)
        self.lib.orc_books_load(ptr(np.ascontiguousarray(books_f16), u16p), nb, en, 8, ptr(b, fp), ptr(bt, fp))
        return b, bt

    def lutb(self, booksT, x, cb_base, order, stages=3, entries=256, vec_dim=8):
        nv = x.size // vec_dim
        lut = np.zeros((nv, stages, entries), np.float32)
        self.lib.orc_lutb(ptr(lut, fp), ptr(booksT, fp), ptr(np.ascontiguousarray(x, np.float32), fp),
                          cb_base, stages, entries, vec_dim, 0, nv, order)
        return lut

    def vq_rows(self, idx_bytes, scale, lut, M, nv):
        y = np.zeros(M, np.float32)
        ib = np.frombuffer(idx_bytes, np.uint8)
        self.lib.orc_vq_rows(ptr(y, fp), ptr(ib, u8p), ptr(np.ascontiguousarray(scale, np.uint16), u16p),
                             ptr(lut, fp), 0, M, nv, 3, 256)
        return y

    def dequant(self, idx_bytes, scale, books, cb_base, M, N):
        W = np.zeros((M, N), np.float32)
        ib = np.frombuffer(idx_bytes, np.uint8)
        self.lib.orc_dequant(ptr(W, fp), ptr(ib, u8p), ptr(np.ascontiguousarray(scale, np.uint16), u16p),
                             ptr(books, fp), cb_base, M, N, 3, 256, 8)
        return W

    def mvq_rows(self, t, x, order):
        y = np.zeros(t.rows, np.float32)
        bits = {2: 8, 3: 4, 7: 3}[t.fmt]
        self.lib.orc_mvq_rows(ptr(y, fp), ptr(t.q, i8p), ptr(t.qs, u16p), ptr(np.ascontiguousarray(x, np.float32), fp),
                              0, t.rows, t.cols, t.group, bits, t.rowbytes, order)
        return y

    def matvec_f32(self, W, x):
        y = np.zeros(W.shape[0], np.float32)
        self.lib.orc_matvec_f32(ptr(y, fp), ptr(np.ascontiguousarray(W, np.float32), fp),
                                ptr(np.ascontiguousarray(x, np.float32), fp), W.shape[0], W.shape[1])
        return y

    def router_scores(self, score_func, logits):
        logits = np.ascontiguousarray(logits, np.float32)
        s = np.zeros_like(logits)
        self.lib.orc_router_scores(score_func, ptr(logits, fp), ptr(s, fp), logits.size)
        return s

    def act_pair(self, g, u):
        g = np.array(g, np.float32)
        self.lib.orc_act_pair(ptr(g, fp), ptr(np.ascontiguousarray(u, np.float32), fp), g.size)
        return g

    def route(self, logits, bias, E, K, score_func, renorm, scale, n_group=1, topk_group=1):
        c = OrcRouteCfg(E, K, score_func, renorm, scale, n_group, topk_group)
        logits = np.ascontiguousarray(logits, np.float32)
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        sc = np.zeros(E, np.float32)
        rc = self.lib.orc_route(C.byref(c), ptr(logits, fp), ptr(bias, fp), ptr(sc, fp), ptr(idx, i32p), ptr(w, fp))
        return rc, idx, w, sc

    def moe(self, layer, order, recs=None):
        """Builds the OrcMoe struct for a records.Layer; keeps the buffers
        alive on the returned object."""
        return _OrcLayer(self, layer, order, recs)


def _tensor(t):
    if t.rows == 0:
        return OrcTensor(0, 0, 0, 0, None, None, 0)
    return OrcTensor(t.fmt, t.rows, t.cols, t.group, t.q.ctypes.data_as(C.c_void_p),
                     ptr(t.qs, u16p) if t.qs is not None else None, t.rowbytes)


class _OrcLayer:
    def __init__(self, orc, L, order, recs=None):
        self.orc, self.L = orc, L
        _, self.booksT = orc.books(L.books_f16)
        self.rec_bufs = [np.frombuffer(r, np.uint8) for r in (recs if recs is not None else L.records)]
        self.rec_ptrs = (u8p * L.E)(*[ptr(b, u8p) for b in self.rec_bufs])
        self.bias = L.bias
        self.m = OrcMoe(L.H, L.E, L.K, L.I, L.n_shared, L.score_func, L.renorm, L.routed_scale,
                        L.n_group, L.topk_group, getattr(L, "stages", 3), getattr(L, "entries", 256), 8,
                        order, _tensor(L.router),
                        ptr(L.bias, fp) if L.bias is not None else None,
                        _tensor(L.sh[0]), _tensor(L.sh[1]), _tensor(L.sh[2]),
                        ptr(self.booksT, fp), L.n_books, self.rec_ptrs, L.rec_bytes)

    def layer(self, x):
        L = self.L
        out = np.zeros(L.H, np.float32)
        idx = np.zeros(L.K, np.int32)
        w = np.zeros(L.K, np.float32)
        lg = np.zeros(L.E, np.float32)
        rc = self.orc.lib.orc_moe_layer(C.byref(self.m), ptr(np.ascontiguousarray(x, np.float32), fp),
                                        ptr(out, fp), ptr(idx, i32p), ptr(w, fp), ptr(lg, fp))
        return rc, out, idx, w, lg

    def layer_mt(self, x, nthreads):
        L = self.L
        out = np.zeros(L.H, np.float32)
        idx = np.zeros(L.K, np.int32)
        w = np.zeros(L.K, np.float32)
        rc = self.orc.lib.orc_moe_layer_mt(C.byref(self.m), ptr(np.ascontiguousarray(x, np.float32), fp),
                                           ptr(out, fp), ptr(idx, i32p), ptr(w, fp), nthreads)
        return rc, out, idx, w

    def apply(self, X, idx, w, chunk):
        L = self.L
        X = np.ascontiguousarray(X, np.float32).reshape(-1, L.H)
        T = X.shape[0]
        out = np.zeros((T, L.H), np.float32)
        rc = self.orc.lib.orc_moe_apply(C.byref(self.m), ptr(X, fp), T,
                                        ptr(np.ascontiguousarray(idx, np.int32), i32p),
                                        ptr(np.ascontiguousarray(w, np.float32), fp), int(chunk), ptr(out, fp))
        return rc, out

    def logits(self, X):
        L = self.L
        X = np.ascontiguousarray(X, np.float32).reshape(-1, L.H)
        out = np.zeros((X.shape[0], L.E), np.float32)
        self.orc.lib.orc_router_logits(C.byref(self.m), ptr(X, fp), X.shape[0], ptr(out, fp))
        return out

    def chunk(self, X):
        L = self.L
        T = X.shape[0]
        out = np.zeros((T, L.H), np.float32)
        idx = np.zeros((T, L.K), np.int32)
        w = np.zeros((T, L.K), np.float32)
        rc = self.orc.lib.orc_moe_chunk(C.byref(self.m), ptr(np.ascontiguousarray(X, np.float32), fp), T,
                                        ptr(out, fp), ptr(idx, i32p), ptr(w, fp))
        return rc, out, idx, w


class RefTensor(C.Structure):
    _fields_ = [("fmt", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("group", C.c_int),
                ("q", C.c_void_p), ("qs", u16p), ("rowbytes", C.c_size_t)]


class Ref:
    """The reference engine's own functions, compiled from its sources."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        _sig(L, "ref_init", C.c_int, [])
        _sig(L, "ref_set_order", None, [C.c_int])
        _sig(L, "ref_set_index_bits", None, [C.c_int])
        _sig(L, "ref_set_stages", None, [C.c_int])
        _sig(L, "ref_vq_rows", None, [fp, u8p, u16p, fp, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "ref_lutb", None, [fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int])
        _sig(L, "ref_vq_quant_lut", None, [fp, C.c_int, C.c_int, C.c_int, i8p, fp])
        _sig(L, "ref_vq_rows_p6", None, [fp, u8p, u16p, i8p, fp, C.c_int, C.c_int])
        _sig(L, "ref_vq_p6_fast", C.c_int, [])
        _sig(L, "ref_mvq_rows", None, [fp, i8p, u16p, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_size_t])
        _sig(L, "ref_matvec_f32", None, [fp, fp, fp, C.c_int, C.c_int])
        _sig(L, "ref_router_scores", None, [C.c_int, fp, fp, C.c_int])
        _sig(L, "ref_act_pair", None, [fp, fp, C.c_int])
        _sig(L, "ref_expf", C.c_float, [C.c_float])
        rt = C.POINTER(RefTensor)
        _sig(L, "ref_moe", C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                     rt, fp, rt, rt, rt, fp, C.c_int, u8p, C.c_size_t, fp, C.c_int, fp, i32p, fp])
        _sig(L, "ref_moe_time", C.c_double, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                             C.c_float, rt, fp, rt, rt, rt, fp, C.c_int, u8p, C.c_size_t, fp,
                                             C.c_int, C.c_int, fp])
        _sig(L, "ref_ecache_run", C.c_int, [C.c_int, C.c_int, C.c_int, i32p, C.c_int, i32p,
                                            C.POINTER(C.c_uint64)])
        _sig(L, "ref_ecache_usage", None, [C.c_char_p, C.c_char_p])
        _sig(L, "ref_ecache_warmed", C.c_int, [])
        self.isa = L.ref_init()

    def vq_quant_lut(self, lut, nv, stages=4, entries=64):
        lut = np.ascontiguousarray(lut, np.float32)
        q = np.zeros(nv * stages * entries, np.int8)
        sc = np.zeros((nv + 31) // 32, np.float32)
        self.lib.ref_vq_quant_lut(ptr(lut, fp), nv, stages, entries, ptr(q, i8p), ptr(sc, fp))
        return q, sc

    def vq_rows_p6(self, idx, scale, lut8, lscale, M, nv):
        """The engine's vq_rows_p6 slot for the current order."""
        idx = np.ascontiguousarray(idx, np.uint8)
        scale = np.ascontiguousarray(scale, np.uint16)
        lut8 = np.ascontiguousarray(lut8, np.int8)
        lscale = np.ascontiguousarray(lscale, np.float32)
        y = np.zeros(M, np.float32)
        self.lib.ref_vq_rows_p6(ptr(y, fp), ptr(idx, u8p), ptr(scale, u16p), ptr(lut8, i8p), ptr(lscale, fp), M, nv)
        return y

    def ecache_run(self, ops, n_slots, depth, policy, warm=None, save=None):
        """The engine's own src/ecache.c on a cache script, reads landing by
        the next demand get: (outputs, [hits, misses, evictions,
        prefetched, spec_issued, reads]).  warm / save: usage files read
        after init / written after the script (ecache_warmed() then says
        how many the warm loaded)."""
        self.lib.ref_ecache_usage(os.fsencode(warm) if warm else None, os.fsencode(save) if save else None)
        a = np.ascontiguousarray(ops, np.int32)
        out = np.zeros(max(len(ops), 1), np.int32)
        st = (C.c_uint64 * 6)()
        k = self.lib.ref_ecache_run(n_slots, depth, policy, ptr(a, i32p), len(ops), ptr(out, i32p), st)
        self.lib.ref_ecache_usage(None, None)
        if k < 0:
            raise RuntimeError("ref_ecache_run failed")
        return [int(v) for v in out[:k]], list(st)

    def ecache_warmed(self):
        return self.lib.ref_ecache_warmed()

    def set_order(self, order):
        self.lib.ref_set_order(order)

    def lutb(self, booksT, x, cb_base, stages=3, entries=256):
        nv = x.size // 8
        lut = np.zeros((nv, stages, entries), np.float32)
        self.lib.ref_lutb(ptr(lut, fp), ptr(np.ascontiguousarray(booksT, np.float32), fp),
                          ptr(np.ascontiguousarray(x, np.float32), fp), cb_base, stages, entries, 8, nv)
        return lut

    def vq_rows(self, idx_bytes, scale, lut, M, nv):
        y = np.zeros(M, np.float32)
        ib = np.frombuffer(idx_bytes, np.uint8)
        self.lib.ref_vq_rows(ptr(y, fp), ptr(ib, u8p), ptr(np.ascontiguousarray(scale, np.uint16), u16p), ptr(lut, fp), M, nv, 3, 256)
        return y

    def mvq_rows(self, t, x):
        y = np.zeros(t.rows, np.float32)
        bits = {2: 8, 3: 4, 7: 3}[t.fmt]
        self.lib.ref_mvq_rows(ptr(y, fp), ptr(t.q, i8p), ptr(t.qs, u16p), ptr(np.ascontiguousarray(x, np.float32), fp),
                              t.rows, t.cols, t.group, bits, t.rowbytes)
        return y

    def matvec_f32(self, W, x):
        y = np.zeros(W.shape[0], np.float32)
        self.lib.ref_matvec_f32(ptr(y, fp), ptr(np.ascontiguousarray(W, np.float32), fp),
                                ptr(np.ascontiguousarray(x, np.float32), fp), W.shape[0], W.shape[1])
        return y

    def router_scores(self, score_func, logits):
        logits = np.ascontiguousarray(logits, np.float32)
        s = np.zeros_like(logits)
        self.lib.ref_router_scores(score_func, ptr(logits, fp), ptr(s, fp), logits.size)
        return s

    def act_pair(self, g, u):
        g = np.array(g, np.float32)
        self.lib.ref_act_pair(ptr(g, fp), ptr(np.ascontiguousarray(u, np.float32), fp), g.size)
        return g

    @staticmethod
    def _rt(t):
        if t.rows == 0:
            return None
        return C.byref(RefTensor(t.fmt, t.rows, t.cols, t.group, t.q.ctypes.data_as(C.c_void_p),
                                 ptr(t.qs, u16p) if t.qs is not None else None, t.rowbytes))

    def moe_time(self, L, X, booksT, nthreads, bank=None):
        """Seconds the engine's moe_layer takes over the tokens X with its
        pool at nthreads and every routed record resident (one untimed pass
        first); and the last token's output."""
        rt = self._rt
        bank = np.frombuffer(L.bank(), np.uint8) if bank is None else bank
        X = np.ascontiguousarray(X, np.float32)
        out = np.zeros(L.H, np.float32)
        sec = self.lib.ref_moe_time(L.H, L.E, L.K, L.I, L.n_shared, L.score_func, L.renorm, L.routed_scale,
                                    rt(L.router), ptr(L.bias, fp) if L.bias is not None else None,
                                    rt(L.sh[0]), rt(L.sh[1]), rt(L.sh[2]), ptr(booksT, fp), L.n_books,
                                    ptr(bank, u8p), L.rec_bytes, ptr(X, fp), X.shape[0], nthreads, ptr(out, fp))
        return sec, out

    def moe(self, L, X, booksT):
        T = X.shape[0]
        rt = self._rt
        self.lib.ref_set_index_bits(getattr(L, "index_bits", 8))
        self.lib.ref_set_stages(getattr(L, "stages", 3))
        bank = np.frombuffer(L.bank(), np.uint8)
        out = np.zeros((T, L.H), np.float32)
        route = np.zeros((T, L.K), np.int32)
        rw = np.zeros((T, L.K), np.float32)
        rc = self.lib.ref_moe(L.H, L.E, L.K, L.I, L.n_shared, L.score_func, L.renorm, L.routed_scale,
                              rt(L.router), ptr(L.bias, fp) if L.bias is not None else None,
                              rt(L.sh[0]), rt(L.sh[1]), rt(L.sh[2]), ptr(booksT, fp), L.n_books,
                              ptr(bank, u8p), L.rec_bytes, ptr(np.ascontiguousarray(X, np.float32), fp), T,
                              ptr(out, fp), ptr(route, i32p), ptr(rw, fp))
        return rc, out, route, rw
