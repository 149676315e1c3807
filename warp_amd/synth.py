# SPDX-License-Identifier: Apache-2.0
"""Seeded synthetic MoE layers at the benchmark shapes.

Trunk tensors (router, bias, shared expert) are generated with numpy and
quantised as the converter does (Q8G: scale = amax/127, Q4G: amax/7, f16
scales per group of 128, round half to even; tools/convert.py:893-924).
Expert records are generated and VQ3R-encoded on the device
(waste_hip_synth_records) against seeded residual k-means codebooks
(waste_hip_synth_codebooks).  Those live in libwaste_hip_synth.so, beside
the product library and separate from it: test and benchmark data only.
"""
import ctypes as C
import os

import numpy as np

from . import LIB_PATH, WQ_F32, WQ_Q4G, WQ_Q8G, HipError, check

SYNTH_LIB_PATH = os.environ.get("WARP_AMD_SYNTH_LIB") or os.path.join(os.path.dirname(LIB_PATH),
                                                                      "libwaste_hip_synth.so")
# Every symbol include/waste_hip_synth.h declares.
SYNTH_EXPORTS = ["waste_hip_record_bytes", "waste_hip_synth_codebooks", "waste_hip_synth_records"]

# The MoE layer shapes the measurements are quoted on.
CONFIGS = {
    # OLMoE: hidden 2048, 64 experts, softmax top-8, intermediate 1024, no shared
    "olmoe": dict(hidden=2048, n_experts=64, top_k=8, moe_inter=1024, n_shared=0, score_func=1,
                  renorm=0, routed_scale=1.0, n_group=1, topk_group=1, router_fmt=WQ_F32,
                  shared_fmt=None, bias=False, bf16=False),
    # Kimi-Linear-48B: hidden 2304, 256 experts, sigmoid top-8 renormalised,
    # 1 shared, intermediate 1024, router and shared 8-bit
    "kimi": dict(hidden=2304, n_experts=256, top_k=8, moe_inter=1024, n_shared=1, score_func=0,
                 renorm=1, routed_scale=2.446, n_group=1, topk_group=1, router_fmt=WQ_Q8G,
                 shared_fmt=WQ_Q8G, bias=True, bf16=False),
    # DeepSeek-V3: hidden 7168, 256 experts, sigmoid + bias, group-limited
    # top-8 (8 groups, 4 kept), scale 2.5, 1 shared (4-bit), intermediate 2048
    "dsv3": dict(hidden=7168, n_experts=256, top_k=8, moe_inter=2048, n_shared=1, score_func=0,
                 renorm=1, routed_scale=2.5, n_group=8, topk_group=4, router_fmt=WQ_F32,
                 shared_fmt=WQ_Q4G, bias=True, bf16=True),
}


def f16_bits(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def quant_q8g(W, group=128):
    rows, N = W.shape
    ng = (N + group - 1) // group
    Wp = np.zeros((rows, ng * group), np.float32)
    Wp[:, :N] = W
    g = Wp.reshape(rows, ng, group)
    sc = np.maximum(np.abs(g).max(-1, keepdims=True), np.float32(1e-8)) / np.float32(127.0)
    q = np.clip(np.rint(g / sc), -127, 127).astype(np.int8).reshape(rows, ng * group)
    return q, f16_bits(sc.reshape(rows, ng)), ng * group


def quant_q4g(W, group=128):
    rows, N = W.shape
    ng = (N + group - 1) // group
    Wp = np.zeros((rows, ng * group), np.float32)
    Wp[:, :N] = W
    g = Wp.reshape(rows, ng, group)
    sc = np.maximum(np.abs(g).max(-1, keepdims=True), np.float32(1e-8)) / np.float32(7.0)
    q = np.clip(np.rint(g / sc), -8, 7).astype(np.int32).reshape(rows, ng * group)
    nib = (q + 8).astype(np.uint8) & 0x0F
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return packed.view(np.int8), f16_bits(sc.reshape(rows, ng)), ng * group // 2


class Tensor:
    """A trunk tensor: fmt, rows, cols, group, payload, f16 scales, rowbytes."""

    def __init__(self, fmt, rows, cols, group, q, qs, rowbytes):
        self.fmt, self.rows, self.cols, self.group = fmt, rows, cols, group
        self.q, self.qs, self.rowbytes = q, qs, rowbytes

    @staticmethod
    def absent():
        return Tensor(WQ_F32, 0, 0, 0, None, None, 0)

    @staticmethod
    def make(fmt, W):
        rows, cols = W.shape
        if fmt == WQ_F32:
            return Tensor(fmt, rows, cols, 0, np.ascontiguousarray(W, np.float32), None, cols * 4)
        if fmt == WQ_Q8G:
            q, qs, rb = quant_q8g(W)
            return Tensor(fmt, rows, cols, 128, q, qs, rb)
        q, qs, rb = quant_q4g(W)
        return Tensor(fmt, rows, cols, 128, q, qs, rb)


_slib = None


def _sigs():
    """The loaded generator library; raises if it has not been built."""
    global _slib
    if _slib is not None:
        return _slib
    if not os.path.exists(SYNTH_LIB_PATH):
        raise HipError(f"{SYNTH_LIB_PATH} is missing: build it with `python -m warp_amd.build`")
    L = C.CDLL(SYNTH_LIB_PATH)
    L.waste_hip_record_bytes.restype = C.c_size_t
    L.waste_hip_record_bytes.argtypes = [C.c_int, C.c_int]
    L.waste_hip_synth_codebooks.restype = C.c_int
    L.waste_hip_synth_codebooks.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_void_p]
    L.waste_hip_synth_records.restype = C.c_int
    L.waste_hip_synth_records.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                          C.c_int, C.c_int, C.c_void_p, C.c_float, C.c_void_p,
                                          C.c_void_p]
    _slib = L
    return L


def record_bytes(hidden, moe_inter):
    return _sigs().waste_hip_record_bytes(hidden, moe_inter)


def codebooks(seed, hidden, moe_inter):
    b = np.zeros((9, 256, 8), np.uint16)
    check(_sigs().waste_hip_synth_codebooks(seed, hidden, moe_inter, b.ctypes.data), "synth_codebooks")
    return b


def records(seed, layer, hidden, moe_inter, books_f16, e0, n, dst_ptr, std=0.02, raw_ptr=None,
            stream=None):
    b = np.ascontiguousarray(books_f16, np.uint16)
    check(_sigs().waste_hip_synth_records(seed, layer, hidden, moe_inter, 0, b.ctypes.data, e0, n,
                                          dst_ptr, std, raw_ptr, stream), "synth_records")


def trunk(cfg, seed):
    """Router (+ bias) and shared expert tensors for a config, N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    H, E, I = cfg["hidden"], cfg["n_experts"], cfg["moe_inter"]
    router = Tensor.make(cfg["router_fmt"], (rng.standard_normal((E, H), np.float32) * 0.02))
    bias = (rng.standard_normal(E, np.float32) * 0.02) if cfg["bias"] else None
    if cfg["n_shared"]:
        SI = I * cfg["n_shared"]
        fmt = cfg["shared_fmt"]
        sh = [Tensor.make(fmt, rng.standard_normal((SI, H), np.float32) * 0.02),
              Tensor.make(fmt, rng.standard_normal((SI, H), np.float32) * 0.02),
              Tensor.make(fmt, rng.standard_normal((H, SI), np.float32) * 0.02)]
    else:
        sh = None
    return router, bias, sh


def dense(t):
    """A trunk tensor's values as float64 [rows][cols] (F32 or Q8G)."""
    if t.fmt == WQ_F32:
        return np.frombuffer(np.ascontiguousarray(t.q).tobytes(), np.float32).reshape(
            t.rows, t.rowbytes // 4)[:, :t.cols].astype(np.float64)
    if t.fmt == WQ_Q8G:
        q = np.frombuffer(np.ascontiguousarray(t.q).tobytes(), np.int8).reshape(t.rows, t.rowbytes)
        s = np.ascontiguousarray(t.qs).view(np.float16).astype(np.float64).reshape(t.rows, -1)
        W = q[:, :t.cols].astype(np.float64)
        return W * np.repeat(s, t.group, axis=1)[:, :t.cols]
    raise ValueError("dense(): F32 or Q8G trunk tensors")


def zipf_tokens(router, T, seed, s=1.1):
    """Tokens whose router logits make per-expert counts follow Zipf(s).

    Expert e gets popularity p_e ~ rank_e^-s (ranks a seeded permutation, so
    popular experts fall in every group); token t's logits are planted as
    log(p_e / p_max) + Gumbel noise, the Gumbel-max form of drawing top-k
    without replacement with probabilities p (the sigmoid score keeps their
    order).  The token is the exact least-squares preimage of those logits
    under the router (x = W^T (W W^T)^-1 l) plus N(0,1) noise orthogonal to
    the router's rows, so every coordinate still looks like N(0,1) noise.
    Returns float32 [T][H]."""
    rng = np.random.default_rng(seed)
    W = dense(router)
    E, H = W.shape
    rank = rng.permutation(E) + 1
    lp = -s * np.log(rank.astype(np.float64))
    L = (lp - lp.max())[None, :] + rng.gumbel(size=(T, E))
    G = W @ W.T
    X = np.linalg.solve(G, L.T).T @ W                          # W X^T = L^T
    Z = rng.standard_normal((T, H))
    Z -= np.linalg.solve(G, (Z @ W.T).T).T @ W                 # remove the row-space part
    return (X + Z).astype(np.float32)
