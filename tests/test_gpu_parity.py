# SPDX-License-Identifier: Apache-2.0
"""The HIP path against the oracle, through the C ABI, on an MI355X.

Bars (written here, per check):
  dequantised weights          bit-exact (closed form, subnormal books flushed)
  expert ids and weights       bit-exact against the oracle's router on the
                               device's own fp32 logits
  router logits                max rel error 1e-5 (fp32 GEMV, other order)
  layer output                 max rel error 1e-3, on the same
                               routing, fp32 accumulation
  VQ3R batch entry             bit-exact (the engine's exact row order)
"""
import ctypes as C
import sys

import numpy as np
import pytest

from gpu_util import LAYER_RTOL, LOGIT_RTOL, gpu_layer, rel_err, run_forward
from oracle_lib import Oracle
from records import FMT_F32, FMT_Q4G, FMT_Q8G, Layer, Tensor, quant_q3g

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402  (after torch: one HIP runtime per process)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module", autouse=True)
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    name = warp_amd.device_name()
    assert name and "gfx950" in name, f"library reports {name}"
    return name


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


CASES = {
    # name: (H, I, E, K, layer kwargs, bf16 input)
    "olmoe_small": (512, 256, 16, 4, dict(score_func=1, seed=101), False),
    "kimi_small": (768, 256, 32, 8, dict(score_func=0, renorm=1, routed_scale=2.446, bias=True,
                                         n_shared=1, shared_fmt=FMT_Q8G, router_fmt=FMT_Q8G, seed=102), False),
    "dsv3_small": (1024, 256, 64, 8, dict(score_func=0, renorm=1, routed_scale=2.5, bias=True,
                                          n_group=8, topk_group=4, n_shared=1, shared_fmt=FMT_Q4G,
                                          router_fmt=FMT_F32, seed=103, subnormal_books=64), True),
}


def make_case(name, T):
    H, I, E, K, kw, bf16 = CASES[name]
    L = Layer(H, I, E, K, **kw)
    X = L.inputs(T, seed=kw["seed"] + 7)
    if bf16:
        X = (torch.from_numpy(X).to(torch.bfloat16).to(torch.float32)).numpy()
    return L, X, bf16


def check_routing(orc, L, lg, ids, w):
    for t in range(lg.shape[0]):
        rc, oi, ow, _ = orc.route(lg[t], L.bias, L.E, L.K, L.score_func, L.renorm, L.routed_scale,
                                  L.n_group, L.topk_group)
        assert rc == L.K
        assert np.array_equal(oi, ids[t]), f"token {t}: ids {ids[t]} vs oracle {oi}"
        assert np.array_equal(bits(ow), bits(w[t])), f"token {t}: weights differ"


@pytest.mark.parametrize("name", list(CASES))
def test_dequant_bit_exact(orc, name):
    say("test_dequant_bit_exact", name)
    L, _, _ = make_case(name, 1)
    m = gpu_layer(L)
    books, _ = orc.books(L.books_f16)
    for e in (0, L.E - 1):
        for kind, (M, N) in enumerate(L.shapes):
            W = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
            assert m.dequant(e, kind, W.data_ptr()) == 0
            torch.cuda.synchronize()
            off = [48, 48 + L.I * L.H * 3 // 8, 48 + 2 * L.I * L.H * 3 // 8][kind]
            ref = orc.dequant(L.records[e][off:], L.scales[e][kind], books, 3 * kind, M, N)
            assert np.array_equal(bits(W.cpu().numpy()), bits(ref)), (e, kind)
    m.close()


@pytest.mark.parametrize("name", list(CASES))
def test_decode_parity(orc, name):
    say("test_decode_parity", name)
    L, X, bf16 = make_case(name, 1)
    m = gpu_layer(L)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16)
    assert st == 0
    ol = orc.moe(L, 1)
    ref_lg = ol.logits(X)
    assert rel_err(lg, ref_lg) <= LOGIT_RTOL
    check_routing(orc, L, lg, ids, w)
    rc, ref = ol.apply(X, ids, w, chunk=0)
    assert rc == 0
    e = rel_err(y, ref)
    say(f"  {name}: layer rel err {e:.3e}")
    assert e <= LAYER_RTOL
    # the oracle's own end-to-end layer picks the same experts on these inputs
    rc, out, oids, ow, _ = ol.layer(X[0])
    assert np.array_equal(oids, ids[0])
    assert rel_err(y[0], out) <= LAYER_RTOL
    m.close()


@pytest.mark.parametrize("name,T", [("kimi_small", 4), ("dsv3_small", 16), ("olmoe_small", 8)])
def test_chunk_parity(orc, name, T):
    say("test_chunk_parity", name, T)
    L, X, bf16 = make_case(name, T)
    m = gpu_layer(L, max_tokens=T)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16)
    assert st == 0
    ol = orc.moe(L, 1)
    assert rel_err(lg, ol.logits(X)) <= LOGIT_RTOL
    check_routing(orc, L, lg, ids, w)
    rc, ref = ol.apply(X, ids, w, chunk=1)
    assert rc == 0
    e = rel_err(y, ref)
    say(f"  {name} T={T}: layer rel err {e:.3e}")
    assert e <= LAYER_RTOL
    m.close()


def test_route_ties(orc):
    """Duplicated router rows give exactly equal logits: the lowest id must
    win, as the engine's strict-greater scan does."""
    say("test_route_ties")
    for sf, bias, ng, tg in [(0, False, 1, 1), (1, False, 1, 1), (0, True, 4, 2)]:
        L = Layer(256, 64, 32, 8, score_func=sf, renorm=1, routed_scale=1.5, bias=bias,
                  n_group=ng, topk_group=tg, seed=200 + sf)
        W = L.router.q.copy()
        for a, b in [(3, 17), (5, 6), (9, 30), (20, 21), (0, 31)]:
            W[b] = W[a]
        L.router.q = W
        if bias:
            L.bias[6] = L.bias[5]
            L.bias[17] = L.bias[3]
        X = L.inputs(4, seed=7)
        m = gpu_layer(L, max_tokens=4)
        st, y, ids, w, lg = run_forward(torch, m, L, X)
        assert st == 0
        check_routing(orc, L, lg, ids, w)
        m.close()


def _planted_layer(E, K, sf, bias, ng, tg, seed):
    """A layer whose router is the identity (F32, H = E), so each token's
    logits are its input vector exactly: planted ties, signed zeros and
    values far outside the sigmoid's range reach the router unchanged."""
    L = Layer(E, 64, E, K, score_func=sf, renorm=1, routed_scale=2.5, bias=bias,
              n_group=ng, topk_group=tg, seed=seed)
    L.router = Tensor.make(FMT_F32, np.eye(E, dtype=np.float32))
    r = np.random.default_rng(seed)
    if bias:
        L.bias = r.choice(np.array([-0.25, 0.0, 0.125, 0.5], np.float32), E)
    return L, r


@pytest.mark.parametrize("E,K,sf,bias,ng,tg", [
    (64, 8, 0, False, 1, 1), (64, 64, 0, True, 1, 1), (64, 8, 1, False, 1, 1),
    (128, 6, 0, True, 16, 5), (256, 8, 0, True, 8, 4), (256, 8, 1, True, 8, 4),
    (256, 8, 0, True, 64, 8), (512, 8, 0, True, 1, 1), (1024, 16, 0, True, 16, 3),
    (64, 8, 2, False, 1, 1), (256, 8, 2, True, 8, 4)])
def test_route_planted(orc, E, K, sf, bias, ng, tg):
    """Top-k over planted logits: few distinct values (so most experts tie
    with several others), +-0, and +-40 (sigmoid saturates to exactly 0 and
    1), for every lanes-per-expert width of the router kernel and for
    group-limited selection with 1 to 64 groups.  ids and weights are
    bit-exact against the oracle on the device's logits."""
    say("test_route_planted", E, K, sf, bias, ng, tg)
    L, r = _planted_layer(E, K, sf, bias, ng, tg, seed=E + K + sf + ng)
    vals = np.array([-40, -3, -1, -0.5, -0.0, 0.0, 0.5, 1, 2, 3, 40], np.float32)
    X = r.choice(vals, (16, E))
    m = gpu_layer(L, max_tokens=16)
    st, y, ids, w, lg = run_forward(torch, m, L, X)
    m.close()
    assert st == 0
    assert np.array_equal(lg.view(np.uint32) & 0x7fffffff, X.view(np.uint32) & 0x7fffffff)
    check_routing(orc, L, lg, ids, w)


@pytest.mark.parametrize("E,K,bias,ng,tg,T", [(64, 8, False, 1, 1, 1), (256, 8, True, 8, 4, 1),
                                               (256, 8, True, 8, 4, 16)])
def test_route_sqrt_softplus(orc, E, K, bias, ng, tg, T):
    """sqrt-softplus scores (score_func 2) on spread logits (every token a
    different set of values, through the log1pf branch at 30 and below):
    ids and weights bit-exact against the oracle, whose log1pf is the host
    libm's; at T = 1 through the router launch's own routing."""
    say("test_route_sqrt_softplus", E, K, T)
    L, r = _planted_layer(E, K, 2, bias, ng, tg, seed=E + 7 * T)
    X = np.concatenate([r.standard_normal((T, E // 2)) * 6, r.uniform(-40, 40, (T, E - E // 2))],
                       1).astype(np.float32)
    m = gpu_layer(L, max_tokens=T)
    st, y, ids, w, lg = run_forward(torch, m, L, X)
    m.close()
    assert st == 0
    check_routing(orc, L, lg, ids, w)


def test_route_too_few_candidates(orc):
    """Fewer than K experts above the engine's -1e30 floor: the layer
    reports WASTE_HIP_EROUTE and every id is -1 (the engine would index
    score[-1]); the oracle also refuses the token."""
    say("test_route_too_few_candidates")
    L, r = _planted_layer(64, 8, 0, True, 1, 1, seed=5)
    L.bias = np.full(64, -1e31, np.float32)
    L.bias[[3, 9, 40, 41]] = 0.0
    X = r.standard_normal((1, 64)).astype(np.float32)
    m = gpu_layer(L, max_tokens=1)
    st, y, ids, w, lg = run_forward(torch, m, L, X)
    m.close()
    assert st == warp_amd.EROUTE
    assert np.all(ids == -1) and np.all(w == 0)
    rc, _, _, _ = orc.route(lg[0], L.bias, 64, 8, 0, 1, 2.5, 1, 1)
    assert rc < 0


def test_vq3r_batch_bit_exact(orc):
    say("test_vq3r_batch_bit_exact")
    L = Layer(512, 256, 4, 2, seed=300)
    _, bT = orc.books(L.books_f16)
    x = L.inputs(1, seed=301)[0]
    lut = orc.lutb(bT, x, 0, 1)
    rec_bufs = [np.frombuffer(r, np.uint8) for r in L.records]
    jobs, ys = [], []
    for e in range(L.E):
        for kind in (0, 1):
            y = np.zeros(L.I, np.float32)
            ys.append(y)
            off = 48 + kind * (L.I * L.H * 3 // 8)
            sc_off = 48 + 2 * (L.I * L.H * 3 // 8) + L.H * L.I * 3 // 8 + kind * 2 * L.I
            jobs.append(warp_amd.VqJob(y.ctypes.data, rec_bufs[e].ctypes.data, rec_bufs[e].size, off,
                                       sc_off, lut.ctypes.data, lut.nbytes, 0, L.I, L.H // 8, 3, 256))
    arr = (warp_amd.VqJob * len(jobs))(*jobs)
    assert warp_amd.lib().waste_hip_vq3r(arr, len(jobs)) == 0
    k = 0
    for e in range(L.E):
        for kind in (0, 1):
            off = 48 + kind * (L.I * L.H * 3 // 8)
            ref = orc.vq_rows(L.records[e][off:], L.scales[e][kind], lut, L.I, L.H // 8)
            assert np.array_equal(bits(ys[k]), bits(ref)), (e, kind)
            k += 1


def test_unbound_expert_and_bad_records(orc):
    say("test_unbound_expert_and_bad_records")
    L = Layer(256, 64, 8, 8, score_func=1, seed=400)
    m = gpu_layer(L)
    # every expert is selected when K == E: unbinding one must be reported
    assert m.bind_expert(5, None, 0) == 0
    st, *_ = run_forward(torch, m, L, L.inputs(1))
    assert st == -6
    bad = bytearray(L.records[5])
    bad[6] ^= 1                        # expert id
    assert m.set_expert(5, bytes(bad)) == -4
    m.close()
    m = gpu_layer(L, verify=1)
    bad = bytearray(L.records[3])
    bad[200] ^= 0x10                   # payload byte: only the crc sees it
    assert m.set_expert(3, bytes(bad)) == -5
    m.close()


def test_register_slot(orc):
    """waste_register_hip fills mvq_rows_f32; the engine calls it with the
    whole range (on_device)."""
    say("test_register_slot")
    from oracle_lib import u16p  # noqa: F401
    tab = (C.c_uint8 * 80)()
    name = warp_amd.lib().waste_register_hip(C.cast(tab, C.c_void_p))
    assert name and b"HIP" in name
    fnp = C.cast(C.addressof(tab) + 24, C.POINTER(C.c_void_p)).contents.value
    on_device = C.c_int.from_address(C.addressof(tab) + 56).value
    assert fnp and on_device == 1
    SLOT = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)(fnp)

    class MvqArg(C.Structure):
        _fields_ = [("y", C.c_void_p), ("W", C.c_void_p), ("ws", C.c_void_p), ("xq", C.c_void_p),
                    ("xs", C.c_void_p), ("in_", C.c_int), ("ng", C.c_int), ("group", C.c_int),
                    ("bits", C.c_int), ("rowbytes", C.c_size_t)]
    # The device sums each row in its own order: rows within 1e-5 of the
    # engine's AVX-512 order (not bit-exact).
    for fmt in (FMT_Q8G, FMT_Q4G):
        L = Layer(1024, 512, 2, 1, n_shared=1, shared_fmt=fmt, seed=500 + fmt)
        t = L.sh[0]
        x = L.inputs(1, seed=9)[0]
        y = np.zeros(t.rows, np.float32)
        a = MvqArg(y.ctypes.data, t.q.ctypes.data, t.qs.ctypes.data, None, x.ctypes.data, t.cols,
                   t.cols // 128, 128, 8 if fmt == FMT_Q8G else 4, t.rowbytes)
        SLOT(0, t.rows, C.addressof(a))
        ref = orc.mvq_rows(t, x, 1)
        assert rel_err(y, ref) <= 1e-5
        # the engine drops the device copies before it frees a tensor
        # (src/waste_backend.h:129-131): the next one may reuse its address
        warp_amd.lib().waste_hip_release_host_buffers()
    # Q3G rows (3-bit codes plus a guard byte per row, tools/convert.py:854-892):
    # decoded on the host into int8 rows, only the decoded bytes copied
    rng = np.random.default_rng(77)
    for cols in (1024, 1000):
        W = (rng.standard_normal((384, cols)) * 0.02).astype(np.float32)
        q, qs, rb = quant_q3g(W)
        t = Tensor(7, 384, cols, 128, q.view(np.int8), qs, rb)
        x = rng.standard_normal(cols).astype(np.float32)
        y = np.zeros(t.rows, np.float32)
        a = MvqArg(y.ctypes.data, q.ctypes.data, qs.ctypes.data, None, x.ctypes.data, cols,
                   qs.shape[1], 128, 3, rb)
        SLOT(0, t.rows, C.addressof(a))
        ref = orc.mvq_rows(t, x, 1)
        assert rel_err(y, ref) <= 1e-5, cols
        warp_amd.lib().waste_hip_release_host_buffers()


def test_register_slot_cpu_fallback(orc):
    """A range the device declines (here a group of 16, which its kernels
    do not take) goes to the CPU kernel the table held when the backend
    registered (mvq_rows_cpu, src/model.c:805-812), not to NaN."""
    say("test_register_slot_cpu_fallback")

    class MvqArg(C.Structure):
        _fields_ = [("y", C.c_void_p), ("W", C.c_void_p), ("ws", C.c_void_p), ("xq", C.c_void_p),
                    ("xs", C.c_void_p), ("in_", C.c_int), ("ng", C.c_int), ("group", C.c_int),
                    ("bits", C.c_int), ("rowbytes", C.c_size_t)]
    rows, cols, g = 96, 256, 16
    rng = np.random.default_rng(5)
    W = np.clip(np.rint(rng.standard_normal((rows, cols)) * 40), -127, 127).astype(np.int8)
    ws = (rng.random((rows, cols // g)) * 0.01 + 0.001).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(cols).astype(np.float32)
    calls = []

    def cpu_rows(b, e, p):
        a = C.cast(p, C.POINTER(MvqArg)).contents
        calls.append((b, e))
        out = (C.c_float * rows).from_address(a.y)
        t = Tensor(FMT_Q8G, rows, cols, g, W, ws, cols)
        ref = orc.mvq_rows(t, x, 1)
        for r in range(b, e):
            out[r] = float(ref[r])

    CB = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)
    cb = CB(cpu_rows)
    tab = (C.c_uint8 * 80)()
    C.c_void_p.from_address(C.addressof(tab) + 64).value = C.cast(cb, C.c_void_p).value  # mvq_rows_cpu
    name = warp_amd.lib().waste_register_hip(C.cast(tab, C.c_void_p))
    assert name
    fnp = C.cast(C.addressof(tab) + 24, C.POINTER(C.c_void_p)).contents.value
    SLOT = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)(fnp)
    y = np.full(rows, np.nan, np.float32)
    a = MvqArg(y.ctypes.data, W.ctypes.data, ws.ctypes.data, None, x.ctypes.data, cols, cols // g, g, 8,
               cols)
    SLOT(0, rows, C.addressof(a))
    assert calls == [(0, rows)]
    ref = orc.mvq_rows(Tensor(FMT_Q8G, rows, cols, g, W, ws, cols), x, 1)
    assert np.array_equal(bits(y), bits(ref))
    # registering again with an empty table leaves no CPU kernel behind
    tab2 = (C.c_uint8 * 80)()
    assert warp_amd.lib().waste_register_hip(C.cast(tab2, C.c_void_p))
    warp_amd.lib().waste_hip_release_host_buffers()
