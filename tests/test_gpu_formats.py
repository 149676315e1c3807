# SPDX-License-Identifier: Apache-2.0
"""The other expert formats through the device layer, on an MI355X, through
the C ABI: VQ4P (index_bits 6: four stages of 64 entries, the engine's int8
tables) and VQ2R (two stages of 256 entries, fp32 tables).

  forward, T = 1 and T > 1   ids and weights bit-exact against the oracle's
                             routing on the device logits; the layer output
                             bit-exact against the oracle's experts on that
                             routing (moe_layer's order at T = 1,
                             moe_chunk's above), in both of the engine's
                             orders, when there is no shared expert (every
                             routed row then equals the engine's); with a
                             shared expert (a GEMV in another summation
                             order) within 1e-3
  many pairs                 a VQ4P forward of 40 tokens (its pairs in chunks):
                             bit-exact as above
  full size                  both formats at the C3 expert shape (7168 x
                             2048), batch 1 and 8, both orders: bit-exact
  through the expert cache   forward_cached over a cache smaller than the
                             expert set: outputs bit-exact as above
  records                    a VQ3R record is refused by a VQ4P layer and a
                             VQ4P record by a VQ3R one
  containers                 VQ4P and VQ2R containers opened by
                             waste_hip_container_moe: layers bit-identical
                             to the directly built ones
The oracle's VQ4P and VQ2R layers are pinned by the compiled reference's
moe_layer and moe_chunk (tests/golden/vq_formats.npz).
"""
import ctypes as C
import sys

import numpy as np
import pytest

from gpu_util import LAYER_RTOL, gpu_layer, rel_err, run_forward
from oracle_lib import Oracle, fp, i32p, ptr
from records import FMT_F32, FMT_Q4G, Layer

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402
from test_gpu_parity import bits, check_routing  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


FMT = {"p6": dict(index_bits=6), "r2": dict(stages=2)}
CASES = {
    # OLMoE-like: softmax, no shared expert, fp32 activations
    "p6_softmax": (dict(H=1024, I=512, E=32, K=8, score_func=1, seed=61), False),
    # DeepSeek-V3-like: sigmoid + bias, group limit, a 4-bit shared expert, bf16 activations
    "p6_dsv3": (dict(H=1024, I=512, E=64, K=8, score_func=0, renorm=1, routed_scale=2.5, bias=True, n_group=8,
                     topk_group=4, n_shared=1, shared_fmt=FMT_Q4G, router_fmt=FMT_F32, seed=62), True),
    # ragged: a last scale block of 8 positions (1088 / 8 = 4 * 32 + 8,
    # 576 / 8 = 2 * 32 + 8) and odd row-block counts (17, 9)
    "p6_ragged": (dict(H=1088, I=576, E=16, K=4, score_func=1, seed=66), False),
    "r2_softmax": (dict(H=1024, I=512, E=32, K=8, score_func=1, seed=64), False),
    "r2_ragged": (dict(H=1088, I=576, E=16, K=4, score_func=1, seed=67), False),
    "r2_dsv3": (dict(H=1024, I=512, E=64, K=8, score_func=0, renorm=1, routed_scale=2.5, bias=True, n_group=8,
                     topk_group=4, n_shared=1, shared_fmt=FMT_Q4G, router_fmt=FMT_F32, seed=65), True),
}


def make(name):
    kw, bf16 = CASES[name]
    kw = dict(kw)
    H, I, E, K = kw.pop("H"), kw.pop("I"), kw.pop("E"), kw.pop("K")
    return Layer(H, I, E, K, **FMT[name[:2]], **kw), bf16


def inputs(L, T, seed, bf16):
    X = L.inputs(T, seed=seed)
    return torch.from_numpy(X).to(torch.bfloat16).to(torch.float32).numpy() if bf16 else X


def oracle_apply(orc, L, order, X, ids, w, chunk):
    om = orc.moe(L, order)
    T = X.shape[0]
    out = np.zeros((T, L.H), np.float32)
    rc = orc.lib.orc_moe_apply(C.byref(om.m), ptr(np.ascontiguousarray(X, np.float32), fp), T,
                               np.ascontiguousarray(ids, np.int32).ctypes.data_as(C.POINTER(C.c_int)),
                               ptr(np.ascontiguousarray(w, np.float32), fp), int(chunk), ptr(out, fp))
    assert rc == 0
    return out


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("order", [0, 1])
def test_format_layer_forward(orc, name, order):
    say("test_format_layer_forward", name, order)
    L, bf16 = make(name)
    m = gpu_layer(L, max_tokens=8, p6_order=order)
    for T in (1, 8):
        X = inputs(L, T, 700 + T, bf16)
        st, y, ids, w, lg = run_forward(torch, m, L, X, bf16=bf16)
        assert st == 0
        check_routing(orc, L, lg, ids, w)
        ref = oracle_apply(orc, L, order, X, ids, w, T > 1)
        e = rel_err(y, ref)
        say(f"  T={T}: rel err {e:.3e}, bit-exact {np.array_equal(bits(y), bits(ref))}")
        if L.n_shared:
            assert e <= LAYER_RTOL
        else:
            assert np.array_equal(bits(y), bits(ref)), (T, e)
    m.close()


_FULL = {}


def full_layer(fmt):
    """The DeepSeek-V3 expert shape (hidden 7168, inter 2048), eight experts,
    top-8 (so batch 8 holds 64 pairs), softmax, no shared expert."""
    if fmt not in _FULL:
        _FULL[fmt] = Layer(7168, 2048, 8, 8, score_func=1, seed=81 if fmt == "p6" else 82, **FMT[fmt])
    return _FULL[fmt]


@pytest.mark.parametrize("fmt", ["p6", "r2"])
@pytest.mark.parametrize("order", [0, 1])
def test_format_layer_fullsize(orc, fmt, order):
    """Both formats at the C3 expert shape the bench measures, batch 1 and 8:
    outputs bit-exact against the oracle in both of the engine's orders."""
    say("test_format_layer_fullsize", fmt, order)
    L = full_layer(fmt)
    m = gpu_layer(L, max_tokens=8, p6_order=order)
    for T in (1, 8):
        X = inputs(L, T, 780 + T, False)
        st, y, ids, w, lg = run_forward(torch, m, L, X)
        assert st == 0
        check_routing(orc, L, lg, ids, w)
        ref = oracle_apply(orc, L, order, X, ids, w, T > 1)
        say(f"  T={T}: rel err {rel_err(y, ref):.3e}, bit-exact {np.array_equal(bits(y), bits(ref))}")
        assert np.array_equal(bits(y), bits(ref)), (T, rel_err(y, ref))
    m.close()


@pytest.mark.parametrize("order", [0, 1])
def test_format_layer_many_pairs(orc, order):
    """A VQ4P forward of 40 tokens (320 pairs) runs its pairs in chunks of
    256 and folds their down rows before the combine: bit-exact against the
    oracle's chunk order as at 8 tokens."""
    say("test_format_layer_many_pairs", order)
    L, bf16 = make("p6_softmax")
    m = gpu_layer(L, max_tokens=40, p6_order=order)
    X = inputs(L, 40, 760, bf16)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16=bf16)
    assert st == 0
    check_routing(orc, L, lg, ids, w)
    ref = oracle_apply(orc, L, order, X, ids, w, 1)
    say(f"  T=40: rel err {rel_err(y, ref):.3e}")
    assert np.array_equal(bits(y), bits(ref))
    m.close()


@pytest.mark.parametrize("name", ["p6_softmax", "r2_softmax"])
def test_format_layer_through_cache(orc, name):
    """forward_cached over 12 slots for 32 experts: every miss filled from
    pinned host memory, the outputs as forward()'s."""
    say("test_format_layer_through_cache", name)
    L, bf16 = make(name)
    order = warp_amd.lib().waste_hip_vq_p6_order()
    m = gpu_layer(L, max_tokens=1, records=False, p6_order=order)
    assert m.bind_table([], [], codebook_id=L.cb_base) == 0
    rb = L.rec_bytes
    host = torch.from_numpy(np.frombuffer(L.bank(), np.uint8).copy()).pin_memory()
    cache = warp_amd.ExpertCache(rb, 12 * rb, policy=0, depth=2)
    cache.set_source([host.data_ptr() + e * rb for e in range(L.E)], 1, L.E)
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    for t in range(6):
        X = inputs(L, 1, 900 + t, False)
        xd = torch.from_numpy(X).to(dev)
        y = torch.full((1, L.H), float("nan"), device=dev)
        ids = torch.empty((1, L.K), dtype=torch.int32, device=dev)
        w = torch.empty((1, L.K), device=dev)
        m.forward_cached(cache, 0, xd.data_ptr(), y.data_ptr(), ids_ptr=ids.data_ptr(), w_ptr=w.data_ptr(),
                         stream=s)
        assert m.status(s) == 0
        ref = oracle_apply(orc, L, order, X, ids.cpu().numpy(), w.cpu().numpy(), 0)
        assert np.array_equal(bits(y.cpu().numpy()), bits(ref)), t
    st = cache.stats()
    say(f"  cache: hits {st['hits']} misses {st['misses']}")
    assert st["misses"] >= 12
    cache.close()
    m.close()


def test_format_records_checked(orc):
    """Each layer takes only its own format's records."""
    say("test_format_records_checked")
    L6, _ = make("p6_softmax")
    L2, _ = make("r2_softmax")
    L8 = Layer(L6.H, L6.I, L6.E, L6.K, score_func=1, seed=63)
    m6 = gpu_layer(L6, records=False)
    m2 = gpu_layer(L2, records=False)
    m8 = gpu_layer(L8, records=False)
    assert m6.set_expert(0, L8.records[0]) == warp_amd.ERECORD
    assert m8.set_expert(0, L6.records[0]) == warp_amd.ERECORD
    assert m2.set_expert(0, L8.records[0]) == warp_amd.ERECORD    # the record size differs too
    assert m8.set_expert(0, L2.records[0]) == warp_amd.ERECORD
    assert m6.set_expert(0, L6.records[0]) == 0
    assert m2.set_expert(0, L2.records[0]) == 0
    m2.close()
    # the device-side check of the table path: the wrong format stays unbound
    d8 = torch.from_numpy(np.frombuffer(L8.records[1], np.uint8).copy()).cuda()
    s = torch.cuda.current_stream().cuda_stream
    assert m6.bind_table([1], [d8.data_ptr()], stream=s) == 0
    assert m6.status(s) == warp_amd.ERECORD
    m6.close()
    m8.close()


@pytest.mark.parametrize("fmt", ["p6", "r2"])
def test_format_container_layer(orc, tmp_path, fmt):
    """Two layers (with a shared expert, which the engine's layer always
    reads) written as a VQ4P container (index_bits 6, twelve books a layer)
    or a VQ2R one (two stages, six books) and opened with
    waste_hip_container_moe: outputs bit-identical to the layers built
    directly from the same arrays."""
    say("test_format_container_layer", fmt)
    from container_writer import build, write
    kw, _ = CASES["p6_softmax"]
    nbk = 12 if fmt == "p6" else 6
    Ls = [Layer(kw["H"], kw["I"], kw["E"], kw["K"], score_func=1, seed=70 + r, cb_base=nbk * r, layer=1 + r,
                n_shared=1, shared_fmt=FMT_Q4G, **FMT[fmt]) for r in range(2)]
    manifest, files = build(Ls, n_layers=3, first_dense=1)
    path = write(str(tmp_path / "ctr"), manifest, files)
    ct = warp_amd.Container(path, verify=True)
    c = ct.config()
    assert (c["index_bits"], c["stages"]) == ((6, 4) if fmt == "p6" else (8, 2))
    order = warp_amd.lib().waste_hip_vq_p6_order()
    for r, L in enumerate(Ls):
        mc = ct.moe(1 + r, max_tokens=4)
        md = gpu_layer(L, max_tokens=4, p6_order=order)
        for T in (1, 4):
            X = inputs(L, T, 40 + T, False)
            a = run_forward(torch, mc, L, X)
            b = run_forward(torch, md, L, X)
            assert a[0] == 0 and b[0] == 0
            assert np.array_equal(a[2], b[2])
            assert np.array_equal(bits(a[1]), bits(b[1])), (r, T)
        mc.close()
        md.close()
    ct.close()
