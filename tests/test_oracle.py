# SPDX-License-Identifier: Apache-2.0
"""The oracle against the reference's golden vectors and against what the
mathematics fixes.  CPU only.

Pins, per oracle function (oracle/oracle.c):
  orc_expf          glibc 2.35 values (golden), host libm sample, specials
  orc_f16_*         every one of the 65,536 fp16 patterns vs numpy, with the
                    loader's subnormal flush
  orc_lutb          golden (both orders) + fp64 closed form
  orc_vq_rows       golden + fp64 materialised-W bound
  orc_dequant       closed form recomputed in numpy from the raw indices
  orc_mvq_rows      golden (both orders) + fp64 dequantised matvec bound,
                    Q8G/Q4G (layer goldens) and Q3G (q3g.npz, three widths)
  orc_router_scores golden + numpy formula in fp64
  orc_route         golden ids/weights + brute force tie rule, permutation
                    at K=E, renorm sum, group-limited brute force and its
                    n_group=1 reduction
  orc_act_pair      golden
  orc_moe_layer / orc_moe_chunk   golden (both orders) + fp64 layer bound;
                    VQ4P experts (int8 tables, vq_rows_p6) and VQ2R (two
                    stages) golden in both orders (vq_formats.npz)
  orc_record_check  valid/damaged records, crc32 against zlib
"""
import ctypes
import ctypes.util
import os
import zlib

import numpy as np
import pytest

from golden.make_golden import (CASES, FORMAT_CASES, Q3G_WIDTHS, case_layer, format_case, input_digest, q3g_digest,
                                q3g_inputs)
from oracle_lib import Oracle, fp, i32p, ptr
from records import FMT_F32, Layer, Tensor, quant_q3g, unblock_indices

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def eq_bits(a, b):
    return np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("name", list(CASES))
def test_golden_case(orc, name):
    g = np.load(os.path.join(GOLD, f"{name}.npz"))
    L, X = case_layer(name)
    assert input_digest(L, X) == str(g["digest"]), "inputs drifted from the fixture"
    _, bT = orc.books(L.books_f16)
    for o in (0, 1):
        if o == 1 and int(g["isa"]) != 2:
            continue
        lut = orc.lutb(bT, X[0], L.cb_base, o)
        assert eq_bits(lut, g[f"lut{o}"]), f"lutb order {o}"
        y = orc.vq_rows(L.records[0][48:], L.scales[0][0], lut, L.I, L.H // 8)
        assert eq_bits(y, g[f"vq{o}"]), f"vq_rows order {o}"
        if L.sh[0].rows:
            assert eq_bits(orc.mvq_rows(L.sh[0], X[0], o), g[f"mvq{o}"]), f"mvq order {o}"
        ol = orc.moe(L, o)
        rc, out, idx, w, lg = ol.layer(X[0])
        assert rc == 0
        assert np.array_equal(idx, g[f"layer_ids{o}"])
        assert eq_bits(out, g[f"layer_out{o}"]), f"moe_layer order {o}"
        rc, co, ci, cw = ol.chunk(X)
        assert rc == 0
        assert np.array_equal(ci, g[f"chunk_ids{o}"])
        assert eq_bits(cw, g[f"chunk_w{o}"])
        assert eq_bits(co, g[f"chunk_out{o}"]), f"moe_chunk order {o}"
    assert eq_bits(orc.router_scores(L.score_func, g["logits"]), g["scores"])


def test_golden_scalars(orc):
    g = np.load(os.path.join(GOLD, "scalars.npz"))
    assert eq_bits(orc.act_pair(g["act_g"], g["act_u"]), g["act"])
    ey = np.array([orc.expf(v) for v in g["exp_x"]], np.float32)
    assert eq_bits(ey, g["exp_y"])


def test_golden_sqrt_softplus(orc):
    """score_func 2 (model.c:5478-5484) against the compiled reference's own
    router_scores on special and seeded logits, bit for bit; and the
    formula: sqrt(log1p(exp(l))) in fp64 within 2 ulp below the branch, and
    sqrt(l) exactly above it."""
    g = np.load(os.path.join(GOLD, "scalars.npz"))
    x, y = g["ssp_x"], g["ssp_y"]
    got = orc.router_scores(2, x)
    assert eq_bits(got, y)
    fin = np.isfinite(x)
    hi = fin & (x > 30.0)
    assert eq_bits(got[hi], np.sqrt(x[hi]).astype(np.float32))
    lo = fin & (x <= 30.0) & (x > -80.0)
    want = np.sqrt(np.log1p(np.exp(x[lo].astype(np.float64))))
    ulp = np.abs(np.spacing(want.astype(np.float32))).astype(np.float64)
    assert np.all(np.abs(got[lo].astype(np.float64) - want) <= 2 * ulp)


def test_expf_against_host_libm(orc):
    """On glibc 2.35 (this image) the restatement is glibc's expf bit for bit
    (exhaustively: oracle/expf_check).  Here: 2^20 spread inputs."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    r = np.random.default_rng(0)
    xs = np.concatenate([r.uniform(-104, 89, 1 << 19), r.standard_normal(1 << 19) * 4]).astype(np.float32)
    bad = [x for x in xs[:: 64] if bits(np.float32(libm.expf(float(x)))) != bits(np.float32(orc.expf(float(x))))]
    assert not bad


def test_expf_against_math(orc):
    # within 0.51 ulp of the exact value on a spread of inputs
    r = np.random.default_rng(1)
    xs = r.uniform(-80, 80, 4096).astype(np.float32)
    for x in xs:
        y = np.float32(orc.expf(float(x)))
        exact = np.exp(np.float64(x))
        ulp = np.spacing(np.float32(exact))
        assert abs(np.float64(y) - exact) <= 0.51 * ulp
    assert orc.expf(0.0) == 1.0
    assert orc.expf(float("-inf")) == 0.0
    assert orc.expf(200.0) == float("inf")


def test_f16_conversions_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    s = np.array([orc.lib.orc_f16_scale(int(v)) for v in h], np.float32)
    b = np.array([orc.lib.orc_f16_book(int(v)) for v in h], np.float32)
    e = (h >> 10) & 0x1F
    normal = (e > 0) & (e < 31)
    assert eq_bits(s[normal], ref[normal])
    assert eq_bits(b[normal], ref[normal])
    sub = e == 0
    assert eq_bits(s[sub], ref[sub])                     # scales keep subnormals
    assert np.all(b[sub] == 0) and np.array_equal(np.signbit(b[sub]), np.signbit(ref[sub]))
    top = e == 31                                         # exponent 31 decodes as 2^16 * (1 + m)
    m = (h[top] & 0x3FF).astype(np.float64)
    mag = (2.0 ** 16) * (1 + m / 1024)
    assert np.array_equal(np.abs(s[top]).astype(np.float64), mag)


def test_lutb_closed_form(orc):
    L = Layer(64, 64, 4, 2, seed=3)
    books, bT = orc.books(L.books_f16)
    x = np.random.default_rng(2).standard_normal(64).astype(np.float32)
    for o in (0, 1):
        lut = orc.lutb(bT, x, 0, o)
        exact = np.einsum("vd,scd->vsc", x.reshape(8, 8).astype(np.float64), books[:3].astype(np.float64))
        assert np.max(np.abs(lut - exact)) <= 8 * 2 ** -23 * np.max(np.abs(exact))


def test_dequant_and_apply_closed_form(orc):
    L = Layer(128, 192, 2, 1, seed=4)
    books, bT = orc.books(L.books_f16)
    rec = L.records[1]
    M, N = L.shapes[0]
    W = orc.dequant(rec[48:], L.scales[1][0], books, 0, M, N)
    idx = unblock_indices(rec[48:], M, N)                    # [M][nv][3]
    recon = np.zeros((M, N // 8, 8), np.float32)
    for s in range(3):
        recon = recon + books[s][idx[:, :, s]]
    sc = L.scales[1][0].view(np.float16).astype(np.float32)[:, None]
    assert eq_bits(W, recon.reshape(M, N) * sc)
    assert np.array_equal(idx, L.idx[1][0])
    x = np.random.default_rng(6).standard_normal(N).astype(np.float32)
    for o in (0, 1):
        y = orc.vq_rows(rec[48:], L.scales[1][0], orc.lutb(bT, x, 0, o), M, N // 8)
        exact = W.astype(np.float64) @ x.astype(np.float64)
        bound = 1e-5 * np.abs(W).astype(np.float64) @ np.abs(x).astype(np.float64)
        assert np.all(np.abs(y - exact) <= bound)


def test_q3g_golden(orc):
    """orc_mvq_rows' Q3G branch (3-bit codes at bit 3i, minus 4,
    src/simd.h:101-106) bit for bit against the reference compiled from its
    sources, both fold orders, at three widths (one with a partial last
    group); the inputs are regenerated and checked against the fixture's
    digests first."""
    g = np.load(os.path.join(GOLD, "q3g.npz"))
    for cols in Q3G_WIDTHS:
        t, x = q3g_inputs(cols)
        assert q3g_digest(t, x) == str(g[f"digest_{cols}"]), cols
        for o in (0, 1):
            if o == 1 and int(g["isa"]) != 2:
                continue
            assert eq_bits(orc.mvq_rows(t, x, o), g[f"rows{o}_{cols}"]), (cols, o)


def test_q3g_closed_form(orc):
    """Q3G rows against the quantiser's own signed codes times the f16
    group scales, in fp64: pins the unpacking (bit offsets across byte
    boundaries, the -4 bias) and the scale per 128-column group."""
    rng = np.random.default_rng(41)
    for cols in (1024, 1000):
        W = (rng.standard_normal((64, cols)) * 0.02).astype(np.float32)
        q, qs, rb, codes = quant_q3g(W, codes=True)
        t = Tensor(7, 64, cols, 128, q.view(np.int8), qs, rb)
        x = rng.standard_normal(cols).astype(np.float32)
        ng = qs.shape[1]
        sc = qs.view(np.float16).astype(np.float64).reshape(64, ng, 1)
        Wd = (codes.reshape(64, ng, 128).astype(np.float64) * sc).reshape(64, ng * 128)[:, :cols]
        exact = Wd @ x.astype(np.float64)
        for o in (0, 1):
            y = orc.mvq_rows(t, x, o)
            assert np.all(np.abs(y - exact) <= 1e-5 * (np.abs(Wd) @ np.abs(x))), (cols, o)
        # a planted wrong bias (codes read as unsigned) is caught
        bad = ((codes + 4).reshape(64, ng, 128).astype(np.float64) * sc).reshape(64, ng * 128)[:, :cols] @ x
        assert not np.all(np.abs(orc.mvq_rows(t, x, 1) - bad) <= 1e-5 * (np.abs(Wd) @ np.abs(x)))


def test_mvq_closed_form(orc):
    for fmt in (2, 3):
        L = Layer(512, 64, 2, 1, n_shared=1, shared_fmt=fmt, seed=7)
        t = L.sh[0]
        x = np.random.default_rng(8).standard_normal(t.cols).astype(np.float32)
        ng = t.cols // 128
        if fmt == 2:
            q = t.q.reshape(t.rows, ng, 128).astype(np.float64)
        else:
            p = t.q.view(np.uint8).reshape(t.rows, -1)
            q = np.empty((t.rows, t.cols))
            q[:, 0::2] = (p & 15).astype(np.int32) - 8
            q[:, 1::2] = (p >> 4).astype(np.int32) - 8
            q = q.reshape(t.rows, ng, 128)
        sc = t.qs.view(np.float16).astype(np.float64).reshape(t.rows, ng, 1)
        Wd = (q * sc).reshape(t.rows, t.cols)
        exact = Wd @ x
        for o in (0, 1):
            y = orc.mvq_rows(t, x, o)
            assert np.all(np.abs(y - exact) <= 1e-5 * (np.abs(Wd) @ np.abs(x)))


def brute_topk(v, K, floor=-1e30):
    """Reference semantics by brute force: K passes, strict >, lowest id wins."""
    taken, out = set(), []
    for _ in range(K):
        best, bv = -1, np.float32(floor)
        for e in range(len(v)):
            if e not in taken and v[e] > bv:
                best, bv = e, v[e]
        out.append(best)
        taken.add(best)
    return out


def test_router_scores_formula(orc):
    r = np.random.default_rng(9)
    lg = (r.standard_normal(256) * 2).astype(np.float32)
    sg = orc.router_scores(0, lg)
    assert np.allclose(sg, 1 / (1 + np.exp(-lg.astype(np.float64))), rtol=2e-7, atol=0)
    sm = orc.router_scores(1, lg)
    ref = np.exp(lg.astype(np.float64) - lg.max())
    assert np.allclose(sm, ref / ref.sum(), rtol=1e-5, atol=0)


def test_route_ties_and_permutation(orc):
    r = np.random.default_rng(10)
    for trial in range(200):
        E = int(r.integers(4, 40))
        K = int(r.integers(1, E + 1))
        lg = r.choice(np.array([-1.0, 0.0, 0.5, 1.0], np.float32), E)   # many exact ties
        bias = r.choice(np.array([0.0, 0.25, -0.25], np.float32), E) if trial % 2 else None
        sf = trial % 2
        rc, idx, w, sc = orc.route(lg, bias, E, K, sf, 0, 1.0)
        sel = sc + (bias if bias is not None else np.float32(0))
        assert rc == K
        assert list(idx) == brute_topk(sel.astype(np.float32), K)
        assert eq_bits(w, sc[idx])
        if K == E:
            assert sorted(idx) == list(range(E))


def test_route_renorm_scale(orc):
    r = np.random.default_rng(11)
    lg = r.standard_normal(256).astype(np.float32)
    bias = (r.standard_normal(256) * 0.02).astype(np.float32)
    rc, idx, w, sc = orc.route(lg, bias, 256, 8, 0, 1, 2.5)
    s = np.float32(0)
    for v in sc[idx]:
        s = np.float32(s + v)
    want = (sc[idx] / np.float32(s + np.float32(1e-20))).astype(np.float32) * np.float32(2.5)
    assert eq_bits(w, want)
    assert abs(float(np.sum(w, dtype=np.float64)) - 2.5) < 8 * 2.5 * 2 ** -23


def brute_group(sel, E, G, TG, K):
    gs = E // G
    gscore = []
    for g in range(G):
        p = sel[g * gs:(g + 1) * gs]
        a = brute_topk(p, 2, -np.inf)
        gscore.append(np.float32(p[a[0]] + p[a[1]]))
    keep = brute_topk(np.array(gscore, np.float32), TG, -np.inf)
    masked = np.array([sel[e] if (e // gs) in keep else -np.inf for e in range(E)], np.float32)
    return brute_topk(masked, K)


def test_route_group_limited(orc):
    r = np.random.default_rng(12)
    for trial in range(100):
        G = int(r.choice([2, 4, 8]))
        gs = int(r.choice([2, 4, 8]))
        E = G * gs
        TG = int(r.integers(1, G + 1))
        K = int(r.integers(1, TG * gs + 1))
        lg = r.choice(np.array([-1, -0.5, 0, 0.5, 1], np.float32), E) + \
            (r.standard_normal(E).astype(np.float32) if trial % 3 else 0)
        lg = lg.astype(np.float32)
        bias = (r.choice(np.array([-0.6, 0, 0.3], np.float32), E)).astype(np.float32)
        rc, idx, w, sc = orc.route(lg, bias, E, K, 0, 1, 2.5, G, TG)
        assert rc == K
        assert list(idx) == brute_group((sc + bias).astype(np.float32), E, G, TG, K)
    # n_group = 1 is the plain router exactly
    lg = r.standard_normal(256).astype(np.float32)
    bias = (r.standard_normal(256) * 0.05).astype(np.float32)
    a = orc.route(lg, bias, 256, 8, 0, 1, 2.5, 1, 1)
    b = orc.route(lg, bias, 256, 8, 0, 1, 2.5, 0, 0)
    assert np.array_equal(a[1], b[1]) and eq_bits(a[2], b[2])
    # all groups kept is the plain router too
    c = orc.route(lg, bias, 256, 8, 0, 1, 2.5, 8, 8)
    assert np.array_equal(a[1], c[1]) and eq_bits(a[2], c[2])


def test_layer_fp64_bound(orc):
    """The whole layer against the materialised weights in fp64, on the
    oracle's own expert ids."""
    L = Layer(256, 128, 8, 3, score_func=0, renorm=1, routed_scale=2.0, bias=True, n_shared=1, seed=21)
    books, _ = orc.books(L.books_f16)
    x = L.inputs(1, seed=22)[0]
    ol = orc.moe(L, 1)
    rc, out, idx, w, lg = ol.layer(x)
    x64 = x.astype(np.float64)
    y = np.zeros(L.H)
    for j, e in enumerate(idx):
        rec = L.records[e]
        Ws = []
        for k, (M, N) in enumerate(L.shapes):
            off = [48, 48 + L.I * L.H * 3 // 8, 48 + 2 * L.I * L.H * 3 // 8][k]
            Ws.append(orc.dequant(rec[off:], L.scales[e][k], books, 3 * k, M, N).astype(np.float64))
        g, u = Ws[0] @ x64, Ws[1] @ x64
        h = g / (1 + np.exp(-g)) * u
        y += float(w[j]) * (Ws[2] @ h)

    def deq(t):
        ng = t.cols // 128
        q = t.q.reshape(t.rows, ng, 128).astype(np.float64)
        return (q * t.qs.view(np.float16).astype(np.float64).reshape(t.rows, ng, 1)).reshape(t.rows, t.cols)
    a, b = deq(L.sh[0]) @ x64, deq(L.sh[1]) @ x64
    y += deq(L.sh[2]) @ (a / (1 + np.exp(-a)) * b)
    assert np.max(np.abs(out - y)) <= 1e-4 * np.max(np.abs(y))


def test_record_check(orc):
    import ctypes as C
    L = Layer(128, 64, 2, 1, seed=30)
    rec = bytearray(L.records[1])

    def check(r, layer=0, expert=1, crc=1):
        buf = (C.c_uint8 * len(r)).from_buffer(r)
        return orc.lib.orc_record_check(buf, len(r), layer, expert, L.I, L.H, 3, L.n_books, crc)
    assert check(rec) == 0
    assert check(rec, expert=0) != 0
    bad = bytearray(rec)
    bad[100] ^= 1
    assert check(bad, crc=0) == 0 and check(bad) == 2
    bad = bytearray(rec)
    bad[0] ^= 1
    assert check(bad) == 1
    payload = bytes(rec[48:48 + 2 * L.I * L.H * 3 // 8 + L.H * L.I * 3 // 8 + 2 * (2 * L.I + L.H)])
    assert orc.lib.orc_crc32((C.c_uint8 * len(payload)).from_buffer_copy(payload), len(payload)) == zlib.crc32(payload)


@pytest.mark.parametrize("name", list(CASES) + ["grouped"])
def test_apply_equals_layer_and_chunk(orc, name):
    """orc_moe_apply, the function every GPU layer test compares against,
    is moe_layer's expert half (chunk 0) and moe_chunk's (chunk 1) bit for
    bit when given their own routing; both of those are pinned to the
    compiled reference's golden outputs above."""
    if name == "grouped":
        L = Layer(512, 128, 64, 8, score_func=0, renorm=1, routed_scale=2.5, bias=True, n_group=8,
                  topk_group=4, n_shared=1, shared_fmt=3, seed=44)
        X = L.inputs(5, seed=45)
    else:
        L, X = case_layer(name)
    for o in (0, 1):
        ol = orc.moe(L, o)
        for t in range(X.shape[0]):
            rc, out, idx, w, _ = ol.layer(X[t])
            assert rc == 0
            rc, out2 = ol.apply(X[t:t + 1], idx[None], w[None], chunk=0)
            assert rc == 0 and eq_bits(out2[0], out), (name, o, t)
        rc, co, ci, cw = ol.chunk(X)
        assert rc == 0
        rc, co2 = ol.apply(X, ci, cw, chunk=1)
        assert rc == 0 and eq_bits(co2, co), (name, o)
        # a planted wrong weight is seen (the comparison is not vacuous)
        cw_bad = cw.copy()
        cw_bad[0, 0] = np.nextafter(cw_bad[0, 0], np.float32(1))
        rc, co3 = ol.apply(X, ci, cw_bad, chunk=1)
        assert not eq_bits(co3, co)


def test_cpu_baseline_same_bits(orc):
    L = Layer(512, 256, 16, 4, score_func=0, renorm=1, routed_scale=2.5, bias=True, n_shared=1,
              shared_fmt=3, seed=40)
    x = L.inputs(1, seed=41)[0]
    ol = orc.moe(L, 1)
    rc, out, idx, w, _ = ol.layer(x)
    for nt in (1, 3, 8):
        rc2, out2, idx2, w2 = ol.layer_mt(x, nt)
        assert rc2 == 0 and np.array_equal(idx, idx2) and eq_bits(out, out2)


@pytest.mark.slow
@pytest.mark.skipif(not os.environ.get("WARP_SLOW"), reason="exhaustive expf check: set WARP_SLOW=1")
def test_expf_exhaustive():
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    subprocess.check_call(["make", "-C", os.path.join(root, "oracle"), "expf_check"])
    out = subprocess.check_output([os.path.join(root, "oracle", "expf_check")]).decode()
    assert "mismatches 0" in out


def test_device_log1pf_sampled():
    """The device's log1pf (warp_amd/csrc/hip/log1pf.h, compiled for the
    host) against the host libm, bit for bit, on every 4099th float (about
    a million inputs); WARP_SLOW=1 runs all of them."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    subprocess.check_call(["make", "-s", "-C", os.path.join(root, "oracle"), "log1pf_check"])
    stride = "1" if os.environ.get("WARP_SLOW") else "4099"
    out = subprocess.check_output([os.path.join(root, "oracle", "log1pf_check"), stride]).decode()
    assert " 0 differ" in out, out


@pytest.mark.parametrize("name", list(FORMAT_CASES))
def test_format_layer_golden(orc, name):
    """orc_moe_layer and orc_moe_chunk on VQ4P experts (index_bits 6: the
    gate/up/down tables quantised to int8 per 32 positions, the rows
    through vq_rows_p6) and on VQ2R experts (two stages of 256 entries)
    against the compiled reference's moe_layer and moe_chunk, bit for bit
    in both orders."""
    g = np.load(os.path.join(GOLD, "vq_formats.npz"))
    L, X = format_case(name)
    assert input_digest(L, X) == str(g[f"{name}_digest"])
    for o in (0, 1):
        if o == 1 and int(g["isa"]) != 2:
            continue
        om = orc.moe(L, o)
        rc, out, idx, w, lg = om.layer(X[0])
        assert rc == 0
        assert np.array_equal(idx, g[f"{name}_layer_ids{o}"])
        assert np.array_equal(out.view(np.uint32), g[f"{name}_layer_out{o}"].view(np.uint32)), (name, o)
        T = X.shape[0]
        oc = np.zeros((T, L.H), np.float32)
        ids = np.zeros((T, L.K), np.int32)
        ww = np.zeros((T, L.K), np.float32)
        rc = orc.lib.orc_moe_chunk(ctypes.byref(om.m), ptr(np.ascontiguousarray(X), fp), T, ptr(oc, fp),
                                   ptr(ids, i32p), ptr(ww, fp))
        assert rc == 0
        assert np.array_equal(ids, g[f"{name}_chunk_ids{o}"])
        assert np.array_equal(ww.view(np.uint32), g[f"{name}_chunk_w{o}"].view(np.uint32))
        assert np.array_equal(oc.view(np.uint32), g[f"{name}_chunk_out{o}"].view(np.uint32)), (name, o)
