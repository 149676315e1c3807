# SPDX-License-Identifier: Apache-2.0
"""warp_amd — the MI355X (gfx950) backend for WARP's MoE expert path.

The product is the C-ABI library libwaste_hip.so (include/waste_hip.h).
This module is its Python mirror: ctypes bindings plus MoeLayer, a thin
owner of one waste_hip_moe handle, used by the tests and bench.py.  Device
buffers are passed as integer addresses (e.g. torch tensors' data_ptr()).

There is no fallback: without the built library, or without a gfx950
device, everything here raises.
"""
import ctypes as C
import os

import numpy as np

# WARP_AMD_LIB names another build of the same library (an A/B comparison);
# the default is the in-tree build.
LIB_PATH = os.environ.get("WARP_AMD_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                          "libwaste_hip.so")

WQ_F32, WQ_Q8G, WQ_Q4G, WQ_VQ3R = 0, 2, 3, 4
SCORE_SIGMOID, SCORE_SOFTMAX, SCORE_SQRTSOFTPLUS = 0, 1, 2

ERRORS = {0: "ok", -1: "EINVAL", -2: "ENODEV", -3: "ENOMEM", -4: "ERECORD", -5: "ECRC",
          -6: "EUNBOUND", -7: "EROUTE", -8: "EDEVICE", -9: "ERANGE", -10: "ETIMEOUT",
          -11: "ESCRATCH", -12: "EFORMAT", -13: "EIO"}

OK, EINVAL, ENODEV, ENOMEM, ERECORD, ECRC, EUNBOUND, EROUTE, EDEVICE, ERANGE, ETIMEOUT, ESCRATCH = \
    0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11
EFORMAT, EIO = -12, -13
CT_RECORDS, CT_GROUP_LIMIT = 1, 2

# Every symbol include/waste_hip.h declares (include/waste_hip_synth.h's are
# in libwaste_hip_synth.so: warp_amd.synth).
EXPORTS = ["waste_hip_device_name", "waste_register_hip", "waste_hip_release_host_buffers",
           "waste_hip_vq3r", "waste_hip_moe_create", "waste_hip_moe_destroy",
           "waste_hip_moe_set_router", "waste_hip_moe_set_shared", "waste_hip_moe_set_codebooks",
           "waste_hip_moe_set_expert", "waste_hip_moe_bind_expert", "waste_hip_moe_forward",
           "waste_hip_moe_status", "waste_hip_moe_bytes", "waste_hip_moe_dequant",
           "waste_hip_moe_profile", "waste_hip_moe_profile_read",
           "waste_hip_moe_route", "waste_hip_moe_experts", "waste_hip_moe_bind_table",
           "waste_hip_moe_predict", "waste_hip_moe_set_lookahead_groups", "waste_hip_moe_forward_cached",
           "waste_hip_moe_forward_static", "waste_hip_moe_static_bytes",
           "waste_hip_ecache_create", "waste_hip_ecache_destroy", "waste_hip_ecache_set_source",
           "waste_hip_ecache_hint", "waste_hip_ecache_prefetch", "waste_hip_ecache_get",
           "waste_hip_ecache_hold", "waste_hip_ecache_release", "waste_hip_ecache_admit",
           "waste_hip_ecache_resident_mask", "waste_hip_ecache_resident_all",
           "waste_hip_ecache_stats", "waste_hip_ecache_slot", "waste_hip_ecache_n_slots",
           "waste_hip_ecache_sync", "waste_hip_moe_set_codebooks_at",
           "waste_hip_container_open", "waste_hip_container_close", "waste_hip_container_config",
           "waste_hip_container_bank", "waste_hip_container_codebooks", "waste_hip_container_read_expert",
           "waste_hip_container_read_bank", "waste_hip_container_error", "waste_hip_container_tensor",
           "waste_hip_container_moe", "waste_hip_crc32", "waste_hip_ecache_save_usage",
           "waste_hip_ecache_warm", "waste_hip_vq_quant_lut", "waste_hip_vq_rows_p6",
           "waste_hip_vq_p6_order"]

STAGES = ["router_shared_gate_up", "route", "routed_gate_up", "swiglu", "routed_down",
          "shared_down", "combine"]


class HipError(RuntimeError):
    pass


class MoeCfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
                ("moe_inter", C.c_int), ("n_shared", C.c_int), ("score_func", C.c_int),
                ("renorm", C.c_int), ("routed_scale", C.c_float), ("n_group", C.c_int),
                ("topk_group", C.c_int), ("layer", C.c_int), ("max_tokens", C.c_int),
                ("verify_records", C.c_int), ("prefill_min_tokens", C.c_int),
                ("index_bits", C.c_int), ("p6_order", C.c_int), ("stages", C.c_int)]


class HipTensor(C.Structure):
    _fields_ = [("fmt", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("group", C.c_int),
                ("q", C.c_void_p), ("qs", C.c_void_p), ("rowbytes", C.c_size_t)]


class MoeProf(C.Structure):
    _fields_ = [("forwards", C.c_int), ("ms", C.c_float * 7)]


class EcacheCounts(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("evictions", C.c_uint64),
                ("prefetched", C.c_uint64), ("spec_issued", C.c_uint64), ("reads", C.c_uint64),
                ("bytes_read", C.c_uint64), ("spec_used", C.c_uint64), ("spec_wasted", C.c_uint64)]


class ContainerCfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "vocab", "n_experts", "top_k", "moe_inter",
                                       "n_shared", "first_dense", "latent_dim", "score_func", "renorm")] + \
               [("routed_scale", C.c_float)] + \
               [(n, C.c_int) for n in ("n_group", "topk_group", "stages", "vec_dim", "entries", "index_bits",
                                       "index_block", "n_books", "n_tensors")] + \
               [("prefix", C.c_char * 64)]


class VqJob(C.Structure):
    """waste_vq_job (src/waste_metal.h:31-40)."""
    _fields_ = [("y", C.c_void_p), ("rec", C.c_void_p), ("rec_bytes", C.c_size_t),
                ("idx_off", C.c_uint32), ("sc_off", C.c_uint32), ("lut", C.c_void_p),
                ("lut_bytes", C.c_size_t), ("lut_off", C.c_uint32), ("m", C.c_int),
                ("nv", C.c_int), ("stages", C.c_int), ("entries", C.c_int)]


_lib = None


def lib():
    """The loaded C-ABI library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipError(f"{LIB_PATH} is missing: build it with `python -m warp_amd.build`")
    L = C.CDLL(LIB_PATH)
    vp, i, ip = C.c_void_p, C.c_int, C.POINTER(C.c_int)
    sig = {
        "waste_hip_device_name": (C.c_char_p, []),
        "waste_register_hip": (C.c_char_p, [vp]),
        "waste_hip_release_host_buffers": (None, []),
        "waste_hip_vq3r": (i, [vp, i]),
        "waste_hip_moe_create": (i, [C.POINTER(MoeCfg), C.POINTER(vp)]),
        "waste_hip_moe_destroy": (None, [vp]),
        "waste_hip_moe_set_router": (i, [vp, C.POINTER(HipTensor), vp]),
        "waste_hip_moe_set_shared": (i, [vp, C.POINTER(HipTensor), C.POINTER(HipTensor), C.POINTER(HipTensor)]),
        "waste_hip_moe_set_codebooks": (i, [vp, vp, i]),
        "waste_hip_moe_set_expert": (i, [vp, i, vp, C.c_size_t]),
        "waste_hip_moe_bind_expert": (i, [vp, i, vp, C.c_size_t]),
        "waste_hip_moe_forward": (i, [vp, vp, i, i, vp, vp, vp, vp, vp]),
        "waste_hip_moe_status": (i, [vp, vp]),
        "waste_hip_moe_bytes": (C.c_size_t, [vp, i, i]),
        "waste_hip_moe_dequant": (i, [vp, i, i, vp, vp]),
        "waste_hip_moe_profile": (i, [vp, i]),
        "waste_hip_moe_profile_read": (i, [vp, C.POINTER(MoeProf)]),
        "waste_hip_moe_route": (i, [vp, vp, i, i, vp, vp, vp, vp]),
        "waste_hip_moe_experts": (i, [vp, vp, i, i, vp, vp]),
        "waste_hip_moe_bind_table": (i, [vp, ip, C.POINTER(vp), i, i, vp]),
        "waste_hip_moe_predict": (i, [vp, vp, i, i, vp, vp]),
        "waste_hip_moe_set_lookahead_groups": (i, [vp, i]),
        "waste_hip_moe_forward_cached": (i, [vp, vp, i, vp, i, vp, i, vp, vp, vp, vp]),
        "waste_hip_moe_forward_static": (i, [vp, vp, i, i, vp, vp, vp, vp, vp]),
        "waste_hip_moe_static_bytes": (C.c_size_t, [vp, i]),
        "waste_hip_ecache_create": (i, [C.c_size_t, C.c_size_t, i, i, i, C.POINTER(vp)]),
        "waste_hip_ecache_destroy": (None, [vp]),
        "waste_hip_ecache_set_source": (i, [vp, C.POINTER(vp), i, i]),
        "waste_hip_ecache_hint": (i, [vp, i, ip, i]),
        "waste_hip_ecache_prefetch": (i, [vp, i, ip, i]),
        "waste_hip_ecache_get": (vp, [vp, i, i, vp]),
        "waste_hip_ecache_hold": (vp, [vp, i, i, vp]),
        "waste_hip_ecache_release": (i, [vp, vp]),
        "waste_hip_ecache_admit": (i, [vp, i, i]),
        "waste_hip_ecache_resident_mask": (i, [vp, i, i, C.POINTER(C.c_uint8)]),
        "waste_hip_ecache_resident_all": (i, [vp, i, ip, i]),
        "waste_hip_ecache_stats": (i, [vp, C.POINTER(EcacheCounts)]),
        "waste_hip_ecache_slot": (i, [vp, i, i]),
        "waste_hip_ecache_n_slots": (i, [vp]),
        "waste_hip_ecache_sync": (i, [vp]),
        "waste_hip_moe_set_codebooks_at": (i, [vp, vp, i, i]),
        "waste_hip_container_open": (i, [C.c_char_p, i, C.POINTER(vp)]),
        "waste_hip_container_close": (None, [vp]),
        "waste_hip_container_config": (i, [vp, C.POINTER(ContainerCfg)]),
        "waste_hip_container_bank": (i, [vp, i, ip, ip, C.POINTER(C.c_size_t)]),
        "waste_hip_container_codebooks": (vp, [vp, ip]),
        "waste_hip_container_read_expert": (i, [vp, i, i, vp, C.c_size_t]),
        "waste_hip_container_read_bank": (i, [vp, i, vp, C.c_size_t]),
        "waste_hip_container_error": (i, [vp, ip, ip]),
        "waste_hip_container_tensor": (i, [vp, C.c_char_p, C.POINTER(HipTensor), ip, ip]),
        "waste_hip_container_moe": (i, [vp, i, i, i, i, C.POINTER(vp)]),
        "waste_hip_crc32": (C.c_uint32, [C.c_uint32, vp, C.c_size_t]),
        "waste_hip_ecache_save_usage": (i, [vp, C.c_char_p, C.c_uint64]),
        "waste_hip_ecache_warm": (i, [vp, C.c_char_p]),
        "waste_hip_vq_quant_lut": (i, [vp, i, i, i, vp, vp, vp]),
        "waste_hip_vq_rows_p6": (i, [vp, vp, vp, vp, i, i, i, i, vp, vp]),
        "waste_hip_vq_p6_order": (i, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _lib = L
    return L


def check(rc, what):
    if rc != 0:
        raise HipError(f"{what}: {ERRORS.get(rc, rc)}")


def device_name():
    n = lib().waste_hip_device_name()
    return n.decode() if n else None


def _tensor(t):
    """A HipTensor from an object with fmt/rows/cols/group/q/qs/rowbytes
    (numpy payloads); the caller keeps the arrays alive."""
    return HipTensor(t.fmt, t.rows, t.cols, t.group, t.q.ctypes.data,
                     t.qs.ctypes.data if t.qs is not None else None, t.rowbytes)


class MoeLayer:
    """One device MoE layer (waste_hip_moe)."""

    def __init__(self, *, hidden, n_experts, top_k, moe_inter, n_shared=0, score_func=0,
                 renorm=0, routed_scale=1.0, n_group=1, topk_group=1, layer=0,
                 max_tokens=1, verify_records=0, prefill_min_tokens=0, index_bits=8, p6_order=None,
                 stages=0):
        """index_bits 6: VQ4P experts; stages 2 (index_bits 8): VQ2R.  Their
        tables and rows follow the engine's arithmetic in p6_order (None:
        this host's, as waste_hip_vq_p6_order reports it)."""
        self.L = lib()
        if p6_order is None:
            p6_order = self.L.waste_hip_vq_p6_order() if index_bits == 6 or stages == 2 else 0
        self.cfg = MoeCfg(hidden, n_experts, top_k, moe_inter, n_shared, score_func, renorm,
                          routed_scale, n_group, topk_group, layer, max_tokens, verify_records,
                          prefill_min_tokens, index_bits, p6_order, stages)
        h = C.c_void_p()
        check(self.L.waste_hip_moe_create(C.byref(self.cfg), C.byref(h)), "waste_hip_moe_create")
        self.h = h

    def close(self):
        if self.h:
            self.L.waste_hip_moe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_router(self, t, bias=None):
        ht = _tensor(t)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        check(self.L.waste_hip_moe_set_router(self.h, C.byref(ht), b.ctypes.data if b is not None else None),
              "set_router")

    def set_shared(self, g, u, d):
        if g is None or g.rows == 0:
            check(self.L.waste_hip_moe_set_shared(self.h, None, None, None), "set_shared")
            return
        a, b, c = _tensor(g), _tensor(u), _tensor(d)
        check(self.L.waste_hip_moe_set_shared(self.h, C.byref(a), C.byref(b), C.byref(c)), "set_shared")

    @classmethod
    def _adopt(cls, h):
        """Owns a handle another call created (Container.moe)."""
        self = cls.__new__(cls)
        self.L, self.h, self.cfg = lib(), h, None
        return self

    def set_codebooks(self, books_f16, first=0):
        b = np.ascontiguousarray(books_f16, np.uint16)
        check(self.L.waste_hip_moe_set_codebooks_at(self.h, b.ctypes.data, first, b.shape[0]),
              "set_codebooks")

    def set_expert(self, e, record):
        buf = np.frombuffer(record, np.uint8)
        return self.L.waste_hip_moe_set_expert(self.h, e, buf.ctypes.data, buf.size)

    def bind_expert(self, e, dev_ptr, nbytes):
        return self.L.waste_hip_moe_bind_expert(self.h, e, dev_ptr, nbytes)

    def forward(self, x_ptr, T, y_ptr, ids_ptr=None, w_ptr=None, logits_ptr=None, bf16=False,
                stream=None):
        check(self.L.waste_hip_moe_forward(self.h, x_ptr, int(bf16), T, y_ptr, ids_ptr, w_ptr,
                                           logits_ptr, stream), "forward")

    def status(self, stream=None):
        return self.L.waste_hip_moe_status(self.h, stream)

    def bytes(self, T, n_distinct):
        return self.L.waste_hip_moe_bytes(self.h, T, n_distinct)

    def profile(self, on):
        check(self.L.waste_hip_moe_profile(self.h, int(on)), "profile")

    def profile_read(self):
        p = MoeProf()
        check(self.L.waste_hip_moe_profile_read(self.h, C.byref(p)), "profile_read")
        return p.forwards, dict(zip(STAGES, list(p.ms)))

    def dequant(self, e, kind, W_ptr, stream=None):
        return self.L.waste_hip_moe_dequant(self.h, e, kind, W_ptr, stream)

    def route(self, x_ptr, T, ids_ptr=None, w_ptr=None, logits_ptr=None, bf16=False, stream=None):
        check(self.L.waste_hip_moe_route(self.h, x_ptr, int(bf16), T, ids_ptr, w_ptr, logits_ptr,
                                         stream), "route")

    def experts(self, x_ptr, T, y_ptr, bf16=False, stream=None):
        check(self.L.waste_hip_moe_experts(self.h, x_ptr, int(bf16), T, y_ptr, stream), "experts")

    def bind_table(self, experts, dev_ptrs, codebook_id=-1, stream=None):
        n = len(experts)
        ids = (C.c_int * max(n, 1))(*experts)
        ptrs = (C.c_void_p * max(n, 1))(*dev_ptrs)
        return self.L.waste_hip_moe_bind_table(self.h, ids, ptrs, n, codebook_id, stream)

    def predict(self, x_ptr, n, ids_ptr, bf16=False, stream=None):
        check(self.L.waste_hip_moe_predict(self.h, x_ptr, int(bf16), n, ids_ptr, stream), "predict")

    def set_lookahead_groups(self, on):
        """predict() within the layer's own group limit (True) or by the
        engine's rule, top n of score + bias over every expert (False)."""
        check(self.L.waste_hip_moe_set_lookahead_groups(self.h, int(bool(on))), "set_lookahead_groups")

    def forward_cached(self, cache, layer, x_ptr, y_ptr, nxt=None, lookahead=0, ids_ptr=None,
                       w_ptr=None, bf16=False, stream=None):
        """One decode token through an ExpertCache (layer: the cache key's
        layer; nxt: the next MoeLayer, whose router makes the lookahead)."""
        check(self.L.waste_hip_moe_forward_cached(self.h, cache.h, layer, nxt.h if nxt else None,
                                                  lookahead, x_ptr, int(bf16), y_ptr, ids_ptr, w_ptr,
                                                  stream), "forward_cached")


def _ids(ids):
    a = (C.c_int * max(len(ids), 1))(*[int(v) for v in ids])
    return a, len(ids)


class ExpertCache:
    """The HBM expert cache (waste_hip_ecache).  dry=True runs the policy
    alone, with no device."""

    def __init__(self, rec_bytes, budget_bytes, *, policy=0, depth=2, dry=False):
        self.L = lib()
        h = C.c_void_p()
        check(self.L.waste_hip_ecache_create(rec_bytes, budget_bytes, policy, depth, int(dry),
                                             C.byref(h)), "waste_hip_ecache_create")
        self.h = h
        self.dry = dry
        self.rec_bytes = rec_bytes
        self._src = None

    def close(self):
        if self.h:
            self.L.waste_hip_ecache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def n_slots(self):
        return self.L.waste_hip_ecache_n_slots(self.h)

    def set_source(self, ptrs, n_layers, n_experts):
        """Host record addresses, [layer][expert] flattened; kept alive here."""
        self._src = (C.c_void_p * len(ptrs))(*ptrs)
        check(self.L.waste_hip_ecache_set_source(self.h, self._src, n_layers, n_experts), "set_source")

    def hint(self, layer, ids):
        a, n = _ids(ids)
        check(self.L.waste_hip_ecache_hint(self.h, layer, a, n), "hint")

    def prefetch(self, layer, ids):
        a, n = _ids(ids)
        check(self.L.waste_hip_ecache_prefetch(self.h, layer, a, n), "prefetch")

    def get(self, layer, expert, stream=None):
        return self.L.waste_hip_ecache_get(self.h, layer, expert, stream)

    def hold(self, layer, expert, stream=None):
        return self.L.waste_hip_ecache_hold(self.h, layer, expert, stream)

    def release(self, stream=None):
        check(self.L.waste_hip_ecache_release(self.h, stream), "release")

    def admit(self, layer, expert):
        return self.L.waste_hip_ecache_admit(self.h, layer, expert)

    def resident_mask(self, layer, n):
        out = (C.c_uint8 * max(n, 1))()
        check(self.L.waste_hip_ecache_resident_mask(self.h, layer, n, out), "resident_mask")
        return [int(v) for v in out[:n]]

    def resident_all(self, layer, ids):
        a, n = _ids(ids)
        return self.L.waste_hip_ecache_resident_all(self.h, layer, a, n)

    def slot(self, layer, expert):
        return self.L.waste_hip_ecache_slot(self.h, layer, expert)

    def stats(self):
        c = EcacheCounts()
        check(self.L.waste_hip_ecache_stats(self.h, C.byref(c)), "stats")
        return {k: int(getattr(c, k)) for k, _ in EcacheCounts._fields_}

    def sync(self):
        check(self.L.waste_hip_ecache_sync(self.h), "sync")

    def save_usage(self, path, tokens):
        return self.L.waste_hip_ecache_save_usage(self.h, os.fsencode(path), tokens)

    def warm(self, path):
        """Records loaded from a usage file (>= 0), or a negative code."""
        return self.L.waste_hip_ecache_warm(self.h, os.fsencode(path))


def crc32(data, crc=0):
    """zlib's crc32 as the library computes it."""
    b = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data)
    return int(lib().waste_hip_crc32(crc, b.ctypes.data if b.size else None, b.nbytes))


class TrunkTensor:
    """A trunk tensor read from a container (copies of its payloads)."""

    def __init__(self, ht, ndim, shape):
        self.fmt, self.rows, self.cols, self.group = ht.fmt, ht.rows, ht.cols, ht.group
        self.rowbytes = ht.rowbytes
        self.shape = tuple(shape[:ndim])
        if ht.fmt == WQ_F32:
            self.q = np.ctypeslib.as_array(C.cast(ht.q, C.POINTER(C.c_float)),
                                           (ht.rows * ht.cols,)).copy().reshape(ht.rows, ht.cols)
            self.qs = None
        else:
            ng = (ht.cols + ht.group - 1) // ht.group
            self.q = np.ctypeslib.as_array(C.cast(ht.q, C.POINTER(C.c_uint8)),
                                           (ht.rows * ht.rowbytes,)).copy().reshape(ht.rows, ht.rowbytes)
            self.qs = np.ctypeslib.as_array(C.cast(ht.qs, C.POINTER(C.c_uint16)),
                                            (ht.rows * ng,)).copy().reshape(ht.rows, ng)


class Container:
    """A WARP container directory opened read-only (waste_hip_container)."""

    def __init__(self, path, verify=False):
        self.L = lib()
        h = C.c_void_p()
        check(self.L.waste_hip_container_open(os.fsencode(path), int(verify), C.byref(h)),
              "waste_hip_container_open")
        self.h = h

    def close(self):
        if self.h:
            self.L.waste_hip_container_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def config(self):
        c = ContainerCfg()
        check(self.L.waste_hip_container_config(self.h, C.byref(c)), "config")
        out = {k: getattr(c, k) for k, _ in ContainerCfg._fields_}
        out["prefix"] = c.prefix.decode()
        return out

    def bank(self, layer):
        """(n_experts, codebook_base, rec_bytes), or None without a bank."""
        n, cb, rb = C.c_int(), C.c_int(), C.c_size_t()
        if self.L.waste_hip_container_bank(self.h, layer, C.byref(n), C.byref(cb), C.byref(rb)):
            return None
        return n.value, cb.value, rb.value

    def codebooks(self):
        n = C.c_int()
        p = self.L.waste_hip_container_codebooks(self.h, C.byref(n))
        c = self.config()
        per = c["entries"] * c["vec_dim"]
        if not n.value:
            return np.zeros((0, c["entries"], c["vec_dim"]), np.uint16)
        a = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), (n.value * per,))
        return a.copy().reshape(n.value, c["entries"], c["vec_dim"])

    def read_expert(self, layer, expert, dst=None):
        """(rc, record bytes as uint8)."""
        b = self.bank(layer)
        rb = b[2] if b else 4096
        buf = np.zeros(rb, np.uint8) if dst is None else dst
        rc = self.L.waste_hip_container_read_expert(self.h, layer, expert, buf.ctypes.data, buf.nbytes)
        return rc, buf

    def read_bank(self, layer, dst):
        """Every record of the layer into dst (an object with .ctypes/.nbytes,
        or an integer address and size as (addr, nbytes))."""
        if isinstance(dst, tuple):
            return self.L.waste_hip_container_read_bank(self.h, layer, dst[0], dst[1])
        return self.L.waste_hip_container_read_bank(self.h, layer, dst.ctypes.data, dst.nbytes)

    def error(self):
        lay, exp = C.c_int(), C.c_int()
        rc = self.L.waste_hip_container_error(self.h, C.byref(lay), C.byref(exp))
        return rc, lay.value, exp.value

    def tensor(self, name):
        ht = HipTensor()
        nd = C.c_int()
        sh = (C.c_int * 4)()
        check(self.L.waste_hip_container_tensor(self.h, name.encode(), C.byref(ht), C.byref(nd), sh),
              f"tensor {name}")
        return TrunkTensor(ht, nd.value, list(sh))

    def moe(self, layer, *, max_tokens=1, prefill_min_tokens=0, records=True, group_limit=False):
        """A MoeLayer for container layer `layer`."""
        h = C.c_void_p()
        flags = (CT_RECORDS if records else 0) | (CT_GROUP_LIMIT if group_limit else 0)
        check(self.L.waste_hip_container_moe(self.h, layer, max_tokens, prefill_min_tokens, flags,
                                             C.byref(h)), "waste_hip_container_moe")
        return MoeLayer._adopt(h)
