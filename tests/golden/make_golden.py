# SPDX-License-Identifier: Apache-2.0
"""Writes tests/golden/*.npz from the reference engine compiled from its own
sources (oracle/_ref/libwasteref.so, built by `make -C oracle` where the
reference tree is present).

Each case is a seeded synthetic layer from tests/records.py.  A fixture
stores the case's configuration, a sha256 of every input byte (so a test can
regenerate the inputs and prove they are the ones the vectors were made
from), and the reference's outputs:

  lut{0,1}      LUT of token 0 against the gate books, portable / AVX-512
  vq{0,1}       vq_rows of expert 0's gate on that LUT
  mvq{0,1}      shared-expert gate matvec (Q8G/Q4G cases)
  scores        router_scores of the oracle's logits of token 0
  layer_out{o}, layer_ids{o}      moe_layer, token 0, order o
  chunk_out{o}, chunk_ids{o}, chunk_w{o}   moe_chunk over all tokens
  act           waste_act_pair_range on seeded vectors
  exp_x, exp_y  glibc expf on 65,536 seeded inputs and the special values
  ssp_x, ssp_y  router_scores, sqrt-softplus, on special and seeded logits

vq4p.npz (VQ4P, 6-bit codes through the engine's int8 LUT):
  lut{o}        LUT of x against four 64-entry books, order o
  q{o}, qs{o}   vq_quant_lut of lut{o}
  rows{o}       the vq_rows_p6 slot of order o on q{o}/qs{o}
  qlut, qq, qsc vq_quant_lut of a planted table (an all-zero block, exact
                halves under a unit inverse, a lone extreme)

vq_formats.npz (whole layers in the other expert formats: moe_layer and
moe_chunk with index_bits 6 (VQ4P: the tables quantised to int8 and the rows
through vq_rows_p6) and with two stages of 256 entries (VQ2R)):
  {case}_digest, {case}_layer_out{o}, {case}_layer_ids{o},
  {case}_chunk_out{o}, {case}_chunk_ids{o}, {case}_chunk_w{o}

q3g.npz (Q3G trunk rows, 3-bit codes plus a guard byte, tools/convert.py:854-892):
  rows{o}_{cols}  mvq_rows of order o on the seeded rows of each width
  digest_{cols}   sha256 of the case's packed rows, scales and x

  python tests/golden/make_golden.py [scalars|vq4p|vq_formats|q3g]
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from records import FMT_F32, FMT_Q4G, FMT_Q8G, Layer  # noqa: E402
from oracle_lib import Oracle, Ref  # noqa: E402

# name -> (H, I, E, K, kwargs, T)
CASES = {
    "softmax_f32": (256, 128, 16, 4, dict(score_func=1, seed=11), 3),
    "sigmoid_q8g": (256, 128, 16, 4, dict(score_func=0, renorm=1, routed_scale=2.446, bias=True,
                                          n_shared=1, shared_fmt=FMT_Q8G, router_fmt=FMT_Q8G, seed=12), 4),
    "sigmoid_q4g": (384, 128, 32, 8, dict(score_func=0, renorm=1, routed_scale=2.5, bias=True,
                                          n_shared=1, shared_fmt=FMT_Q4G, router_fmt=FMT_F32, seed=13,
                                          subnormal_books=40), 3),
}


def case_layer(name):
    H, I, E, K, kw, T = CASES[name]
    L = Layer(H, I, E, K, **kw)
    return L, L.inputs(T, seed=kw["seed"] + 100)


def input_digest(L, X):
    h = hashlib.sha256()
    h.update(L.bank())
    h.update(L.books_f16.tobytes())
    for t in [L.router] + list(L.sh):
        if t.rows:
            h.update(t.q.tobytes())
            if t.qs is not None:
                h.update(t.qs.tobytes())
    if L.bias is not None:
        h.update(L.bias.tobytes())
    h.update(X.tobytes())
    return h.hexdigest()


def main():
    orc, ref = Oracle(), Ref()
    if sys.argv[1:] == ["scalars"]:                 # only scalars.npz
        write_scalars(ref)
        return
    if sys.argv[1:] == ["vq4p"]:                    # only vq4p.npz
        write_vq4p(orc, ref)
        return
    if sys.argv[1:] == ["q3g"]:                     # only q3g.npz
        write_q3g(ref)
        return
    if sys.argv[1:] == ["vq_formats"]:              # only vq_formats.npz
        write_vq_formats(orc, ref)
        return
    if ref.isa != 2:
        print("warning: this host does not run the reference's AVX-512 kernels; order 1 = portable")
    for name in CASES:
        L, X = case_layer(name)
        _, bT = orc.books(L.books_f16)
        out = {"digest": np.array(input_digest(L, X)), "isa": np.array(ref.isa)}
        for o in (0, 1):
            ref.set_order(o)
            lut = ref.lutb(bT, X[0], L.cb_base)
            out[f"lut{o}"] = lut
            out[f"vq{o}"] = ref.vq_rows(L.records[0][48:], L.scales[0][0], lut, L.I, L.H // 8)
            if L.sh[0].rows:
                out[f"mvq{o}"] = ref.mvq_rows(L.sh[0], X[0])
            rc, lo, lr, _ = ref.moe(L, X[:1], bT)
            assert rc == 0, rc
            out[f"layer_out{o}"], out[f"layer_ids{o}"] = lo[0], lr[0]
            rc, co, cr, cw = ref.moe(L, X, bT)
            assert rc == 0, rc
            out[f"chunk_out{o}"], out[f"chunk_ids{o}"], out[f"chunk_w{o}"] = co, cr, cw
        if L.router.fmt == FMT_F32:
            out["logits"] = ref.matvec_f32(L.router.q, X[0])
        else:
            ref.set_order(1)
            out["logits"] = ref.mvq_rows(L.router, X[0])
        out["scores"] = ref.router_scores(L.score_func, out["logits"])
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
        print(name, "written")

    write_scalars(ref)
    write_vq4p(orc, ref)
    write_vq_formats(orc, ref)
    write_q3g(ref)


# VQ4P and VQ2R layers: name -> (H, I, E, K, kwargs, T)
FORMAT_CASES = {
    "p6_softmax": (256, 128, 16, 4, dict(score_func=1, seed=41, index_bits=6), 3),
    "p6_sigmoid_q8g": (256, 128, 16, 4, dict(score_func=0, renorm=1, routed_scale=2.5, bias=True,
                                             n_shared=1, shared_fmt=FMT_Q8G, seed=42, index_bits=6), 4),
    "r2_softmax": (256, 128, 16, 4, dict(score_func=1, seed=51, stages=2), 3),
    "r2_sigmoid_q8g": (256, 128, 16, 4, dict(score_func=0, renorm=1, routed_scale=2.5, bias=True,
                                             n_shared=1, shared_fmt=FMT_Q8G, seed=52, stages=2), 4),
}


def format_case(name):
    H, I, E, K, kw, T = FORMAT_CASES[name]
    L = Layer(H, I, E, K, **kw)
    return L, L.inputs(T, seed=kw["seed"] + 100)


def write_vq_formats(orc, ref):
    out = {}
    for name in FORMAT_CASES:
        L, X = format_case(name)
        _, bT = orc.books(L.books_f16)
        out[f"{name}_digest"] = np.array(input_digest(L, X))
        for o in (0, 1):
            ref.set_order(o)
            rc, lo, lr, _ = ref.moe(L, X[:1], bT)
            assert rc == 0, rc
            out[f"{name}_layer_out{o}"], out[f"{name}_layer_ids{o}"] = lo[0], lr[0]
            rc, co, cr, cw = ref.moe(L, X, bT)
            assert rc == 0, rc
            out[f"{name}_chunk_out{o}"], out[f"{name}_chunk_ids{o}"], out[f"{name}_chunk_w{o}"] = co, cr, cw
    ref.lib.ref_set_index_bits(8)
    out["isa"] = np.array(ref.isa)
    np.savez_compressed(os.path.join(HERE, "vq_formats.npz"), **out)
    print("vq_formats written")


Q3G_WIDTHS = (1024, 1000, 640)


def q3g_inputs(cols, seed=31, rows=96):
    """Seeded Q3G rows of one width (a partial last group when cols is not
    a multiple of 128) and x ~ N(0,1)."""
    from records import Tensor, quant_q3g
    r = np.random.default_rng(seed + cols)
    W = (r.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    q, qs, rb = quant_q3g(W)
    x = r.standard_normal(cols).astype(np.float32)
    return Tensor(7, rows, cols, 128, q.view(np.int8), qs, rb), x


def q3g_digest(t, x):
    h = hashlib.sha256()
    h.update(t.q.tobytes())
    h.update(t.qs.tobytes())
    h.update(x.tobytes())
    return h.hexdigest()


def write_q3g(ref):
    out = {"isa": np.array(ref.isa)}
    for cols in Q3G_WIDTHS:
        t, x = q3g_inputs(cols)
        out[f"digest_{cols}"] = np.array(q3g_digest(t, x))
        for o in (0, 1):
            ref.set_order(o)
            out[f"rows{o}_{cols}"] = ref.mvq_rows(t, x)
    np.savez_compressed(os.path.join(HERE, "q3g.npz"), **out)
    print("q3g written")


def vq4p_inputs(seed=21, M=192, nv=80):
    """A seeded VQ4P matrix: four 64-entry books of 8 dims (fp16 values,
    normal), codes as random bytes (every byte triple is four 6-bit codes),
    f16 row scales, x ~ N(0,1); plus a planted table for the quantiser."""
    r = np.random.default_rng(seed)
    books16 = (r.standard_normal((4, 64, 8)) * [[[0.5]], [[0.2]], [[0.08]], [[0.03]]]).astype(np.float16)
    booksT = np.ascontiguousarray(books16.astype(np.float32).transpose(0, 2, 1)).reshape(-1)
    x = r.standard_normal(nv * 8).astype(np.float32)
    idx = r.integers(0, 256, (M // 64) * nv * 192, dtype=np.uint8)
    scale = (np.abs(r.standard_normal(M)) * 0.02 + 0.005).astype(np.float16).view(np.uint16)
    # planted quantiser blocks (64 positions x 256 entries): block 0 all
    # zeros; block 1 holds +-127 once (inverse exactly 1) and halves
    # (ties to even); the rest seeded
    qlut = (r.standard_normal((64, 256)) * 3).astype(np.float32)
    qlut[:32] = 0.0
    halves = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32)
    qlut[32:64] = r.uniform(-120, 120, (32, 256)).astype(np.float32)
    qlut[32, :8] = halves
    qlut[33, 0] = 127.0
    qlut[40, 5] = -127.0
    return books16, booksT, x, idx, scale, qlut.reshape(-1), M, nv


def write_vq4p(orc, ref):
    books16, booksT, x, idx, scale, qlut, M, nv = vq4p_inputs()
    h = hashlib.sha256()
    for a in (books16, x, idx, scale, qlut):
        h.update(a.tobytes())
    out = {"digest": np.array(h.hexdigest()), "isa": np.array(ref.isa), "p6_fast": np.array(ref.lib.ref_vq_p6_fast())}
    for o in (0, 1):
        ref.set_order(o)
        lut = ref.lutb(booksT, x, 0, stages=4, entries=64)
        q, qs = ref.vq_quant_lut(lut, nv)
        out[f"lut{o}"], out[f"q{o}"], out[f"qs{o}"] = lut, q, qs
        out[f"rows{o}"] = ref.vq_rows_p6(idx, scale, q, qs, M, nv)
    out["qlut"] = qlut
    out["qq"], out["qsc"] = ref.vq_quant_lut(qlut, 64, 4, 64)
    np.savez_compressed(os.path.join(HERE, "vq4p.npz"), **out)
    print("vq4p written")


def write_scalars(ref):
    # activation and expf
    r = np.random.default_rng(5)
    g = (r.standard_normal(4096) * 4).astype(np.float32)
    u = r.standard_normal(4096).astype(np.float32)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 88.0, 88.72283, 88.7229, -87.0, -103.0, -103.97,
                         -104.0, 30.0, -30.0, np.inf, -np.inf, 1e-30, -1e-30, float.fromhex("0x1.04845ep+5"),
                         float.fromhex("-0x1.f8cbb2p+5")], np.float32)
    ex = np.concatenate([specials, (r.standard_normal(65536) * 20).astype(np.float32)])
    ey = np.array([ref.lib.ref_expf(float(v)) for v in ex], np.float32)
    # sqrt-softplus router scores (score_func 2): the branch at 30, the
    # log1pf of tiny and huge arguments, and a seeded spread of logits
    sspec = np.array([0.0, -0.0, 1e-8, -1e-8, 1e-3, -1e-3, 0.5, -0.5, 29.999998, 30.0, 30.000002, -30.0,
                      -80.0, -87.0, -103.0, -104.0, 88.0, 100.0, np.inf, -np.inf], np.float32)
    sx = np.concatenate([sspec, (r.standard_normal(16384) * 8).astype(np.float32),
                         r.uniform(-110, 110, 16384).astype(np.float32)])
    sy = ref.router_scores(2, sx)
    np.savez_compressed(os.path.join(HERE, "scalars.npz"), act_g=g, act_u=u,
                        act=ref.act_pair(g, u), exp_x=ex, exp_y=ey, ssp_x=sx, ssp_y=sy)
    print("scalars written")


if __name__ == "__main__":
    main()
