# SPDX-License-Identifier: Apache-2.0
"""The layer driven through an expert cache, on an MI355X, through the C ABI.

  route + experts          bit-identical to forward (same kernels, split)
  bind_table               bit-identical to set_expert; a record with the
                           wrong header is refused on the device (ERECORD)
  predict                  the lookahead's ids bit-exact against the
                           oracle's predict_next_moe on the device logits
  cache-fed layers         every layer output within 1e-3 of the oracle's
                           moe_layer on the full record set, ids bit-exact,
                           dequantised slot contents bit-exact; the cache's
                           decisions equal its dry replay
"""
import sys

import numpy as np
import pytest

import ecache_script as es
from gpu_util import LAYER_RTOL, gpu_layer, rel_err
from oracle_lib import Oracle
from records import FMT_F32, FMT_Q4G, Layer

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402
from test_gpu_parity import bits, check_routing, make_case  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


def stream():
    return torch.cuda.current_stream().cuda_stream


def dsv3_layer(layer, seed):
    return Layer(1024, 256, 64, 8, score_func=0, renorm=1, routed_scale=2.5, bias=True,
                 n_group=8, topk_group=4, n_shared=1, shared_fmt=FMT_Q4G, router_fmt=FMT_F32,
                 seed=seed, layer=layer)


def bf16_inputs(L, T, seed):
    X = L.inputs(T, seed=seed)
    return torch.from_numpy(X).to(torch.bfloat16).to(torch.float32).numpy()


@pytest.mark.parametrize("T,prefill_min", [(1, 0), (8, 0), (64, 16)])
def test_route_experts_equal_forward(orc, T, prefill_min):
    say("test_route_experts_equal_forward", T)
    L, X, bf16 = make_case("dsv3_small", T)
    m = gpu_layer(L, max_tokens=T, prefill_min=prefill_min)
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(X).to(dev).to(torch.bfloat16)
    outs = []
    for split in (False, True):
        y = torch.full((T, L.H), float("nan"), device=dev)
        ids = torch.empty((T, L.K), dtype=torch.int32, device=dev)
        w = torch.empty((T, L.K), dtype=torch.float32, device=dev)
        if split:
            m.route(xd.data_ptr(), T, ids.data_ptr(), w.data_ptr(), None, bf16=True, stream=stream())
            m.experts(xd.data_ptr(), T, y.data_ptr(), bf16=True, stream=stream())
        else:
            m.forward(xd.data_ptr(), T, y.data_ptr(), ids.data_ptr(), w.data_ptr(), None, bf16=True,
                      stream=stream())
        assert m.status(stream()) == 0
        outs.append((y.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()))
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(bits(outs[0][2]), bits(outs[1][2]))
    # experts() needs the route of the same T first
    m2 = gpu_layer(L, max_tokens=T, prefill_min=prefill_min)
    y = torch.empty((T, L.H), device=dev)
    with pytest.raises(warp_amd.HipError):
        m2.experts(xd.data_ptr(), T, y.data_ptr(), bf16=True, stream=stream())
    m.close()
    m2.close()


def test_bind_table_equals_set_expert(orc):
    say("test_bind_table_equals_set_expert")
    L, X, bf16 = make_case("dsv3_small", 1)
    dev = torch.device("cuda:0")
    ref = gpu_layer(L)
    slab = torch.from_numpy(np.frombuffer(L.bank(), np.uint8).copy()).to(dev)
    base = slab.data_ptr()
    assert base % 256 == 0
    m = gpu_layer(L, records=False)
    xd = torch.from_numpy(X).to(dev).to(torch.bfloat16)

    def run(layer):
        y = torch.full((1, L.H), float("nan"), device=dev)
        ids = torch.empty((1, L.K), dtype=torch.int32, device=dev)
        layer.forward(xd.data_ptr(), 1, y.data_ptr(), ids.data_ptr(), None, None, bf16=True,
                      stream=stream())
        return layer.status(stream()), y.cpu().numpy(), ids.cpu().numpy()

    # the whole table, in two calls of 32, stream-ordered (no host wait)
    for lo in (0, 32):
        es_ = list(range(lo, lo + 32))
        assert m.bind_table(es_, [base + e * L.rec_bytes for e in es_], codebook_id=L.cb_base,
                            stream=stream()) == 0
    st0, y0, i0 = run(ref)
    st1, y1, i1 = run(m)
    assert st0 == 0 and st1 == 0
    assert np.array_equal(i0, i1) and np.array_equal(bits(y0), bits(y1))

    # a record whose header names another expert is refused on the device
    e = int(i1[0, 0])
    wrong = (e + 1) % L.E
    assert m.bind_table([e], [base + wrong * L.rec_bytes], stream=stream()) == 0
    st, y, _ = run(m)
    assert st == warp_amd.ERECORD
    assert m.bind_table([e], [base + e * L.rec_bytes], stream=stream()) == 0
    st, y, _ = run(m)
    assert st == 0 and np.array_equal(bits(y), bits(y1))
    # unbinding a routed expert: its rows are zeros and status says so
    assert m.bind_table([e], [None], stream=stream()) == 0
    st, y, _ = run(m)
    assert st == warp_amd.EUNBOUND
    # host-side argument checks
    assert m.bind_table([1, 1], [base + L.rec_bytes] * 2) == warp_amd.EINVAL
    assert m.bind_table([1], [base + L.rec_bytes + 8]) == warp_amd.EINVAL
    assert m.bind_table([1], [base + L.rec_bytes], codebook_id=L.cb_base + 1) == warp_amd.ERECORD
    m.close()
    ref.close()


@pytest.mark.parametrize("name,n", [("dsv3_small", 6), ("dsv3_small", 64), ("kimi_small", 16),
                                    ("olmoe_small", 5)])
def test_predict_matches_oracle(orc, name, n):
    say("test_predict_matches_oracle", name, n)
    L, X, bf16 = make_case(name, 4)
    m = gpu_layer(L)
    dev = torch.device("cuda:0")
    for t in range(X.shape[0]):
        xd = torch.from_numpy(X[t:t + 1]).to(dev)
        if bf16:
            xd = xd.to(torch.bfloat16)
        lg = torch.empty((1, L.E), device=dev)
        y = torch.empty((1, L.H), device=dev)
        m.forward(xd.data_ptr(), 1, y.data_ptr(), None, None, lg.data_ptr(), bf16=bf16, stream=stream())
        ids = torch.full((64,), -5, dtype=torch.int32, device=dev)
        m.predict(xd.data_ptr(), n, ids.data_ptr(), bf16=bf16, stream=stream())
        assert m.status(stream()) == 0
        got = ids.cpu().numpy()
        want = orc.predict_next(L.score_func, lg.cpu().numpy()[0], L.bias, n)
        k = min(n, L.E)
        assert np.array_equal(got[:k], want), (t, got[:k], want)
        assert np.all(got[k:] == -5)
    m.close()


@pytest.mark.parametrize("name,n", [("dsv3_small", 6), ("dsv3_small", 64), ("olmoe_small", 5)])
def test_predict_grouped_matches_oracle(orc, name, n):
    """With the lookahead in the layer's own group limit: the oracle's
    group-limited route of n (no renorm, scale 1) on the device logits, in
    its order; n capped at the kept groups' experts (dsv3_small: 4 of 8
    groups of 8, so 32), ids past the cap untouched.  A layer without
    groups keeps predict_next_moe's rule."""
    say("test_predict_grouped_matches_oracle", name, n)
    L, X, bf16 = make_case(name, 4)
    m = gpu_layer(L)
    m.set_lookahead_groups(True)
    dev = torch.device("cuda:0")
    for t in range(X.shape[0]):
        xd = torch.from_numpy(X[t:t + 1]).to(dev)
        if bf16:
            xd = xd.to(torch.bfloat16)
        lg = torch.empty((1, L.E), device=dev)
        y = torch.empty((1, L.H), device=dev)
        m.forward(xd.data_ptr(), 1, y.data_ptr(), None, None, lg.data_ptr(), bf16=bf16, stream=stream())
        ids = torch.full((64,), -5, dtype=torch.int32, device=dev)
        m.predict(xd.data_ptr(), n, ids.data_ptr(), bf16=bf16, stream=stream())
        assert m.status(stream()) == 0
        got = ids.cpu().numpy()
        logits = lg.cpu().numpy()[0]
        if L.n_group > 1:
            k = min(n, L.topk_group * (L.E // L.n_group))
            rc, want, _, _ = orc.route(logits, L.bias, L.E, k, L.score_func, 0, 1.0, L.n_group, L.topk_group)
            assert rc == k
        else:
            k = min(n, L.E)
            want = orc.predict_next(L.score_func, logits, L.bias, n)
        assert np.array_equal(got[:k], want), (t, got[:k], want)
        assert np.all(got[k:] == -5)
    m.close()


@pytest.mark.parametrize("n_slots,depth,look,own", [(20, 2, 6, False), (72, 2, 6, True),
                                                   (200, 2, 0, False), (24, 4, 16, True)])
def test_cache_fed_layers(orc, n_slots, depth, look, own):
    """Three layers, 10 tokens, the cache smaller than the expert set: every
    output against the oracle on the full record set.  own: on a stream of
    its own rather than the null stream."""
    say("test_cache_fed_layers", n_slots, depth, look, own)
    if own:
        with torch.cuda.stream(torch.cuda.Stream()):
            _cache_fed_layers(orc, n_slots, depth, look)
    else:
        _cache_fed_layers(orc, n_slots, depth, look)


def _cache_fed_layers(orc, n_slots, depth, look):
    n_layers, T = 3, 10
    dev = torch.device("cuda:0")
    Ls = [dsv3_layer(l, 300 + l) for l in range(n_layers)]
    rec = Ls[0].rec_bytes
    host = torch.empty((n_layers * Ls[0].E, rec), dtype=torch.uint8, pin_memory=True)
    for l, L in enumerate(Ls):
        host[l * L.E:(l + 1) * L.E] = torch.from_numpy(np.frombuffer(L.bank(), np.uint8).reshape(L.E, rec).copy())
    cache = warp_amd.ExpertCache(rec, n_slots * rec, policy=0, depth=depth)
    cache.set_source([host.data_ptr() + i * rec for i in range(n_layers * Ls[0].E)], n_layers, Ls[0].E)
    ms = [gpu_layer(L, records=False) for L in Ls]
    ols = [orc.moe(L, 1) for L in Ls]
    ops = []
    s = stream()
    ids_d = torch.empty((1, 8), dtype=torch.int32, device=dev)
    look_d = torch.empty((64,), dtype=torch.int32, device=dev)
    worst = 0.0
    books = [orc.books(L.books_f16)[0] for L in Ls]
    for t in range(T):
        xs = [bf16_inputs(L, 1, 1000 * t + l) for l, L in enumerate(Ls)]
        for l, (L, m) in enumerate(zip(Ls, ms)):
            xd = torch.from_numpy(xs[l]).to(dev).to(torch.bfloat16)
            lg = torch.empty((1, L.E), device=dev)
            w_d = torch.empty((1, 8), device=dev)
            m.route(xd.data_ptr(), 1, ids_d.data_ptr(), w_d.data_ptr(), lg.data_ptr(), bf16=True, stream=s)
            if look and l + 1 < n_layers:
                ms[l + 1].predict(xd.data_ptr(), look, look_d.data_ptr(), bf16=True, stream=s)
            ids = ids_d.cpu().numpy()[0].tolist()            # waits for the route
            cache.hint(l, ids)
            ops += [es.HINT, l, len(ids)] + ids
            ptrs = []
            for e in ids:
                p = cache.hold(l, e, s)
                assert p, (t, l, e)
                ptrs.append(p)
                ops += [es.HOLD, l, e]
            assert m.bind_table(ids, ptrs, codebook_id=L.cb_base, stream=s) == 0
            y = torch.full((1, L.H), float("nan"), device=dev)
            m.experts(xd.data_ptr(), 1, y.data_ptr(), bf16=True, stream=s)
            if t == T - 1:
                # the slot bytes themselves, through the bound table
                e = ids[0]
                for kind, (M, N) in enumerate(L.shapes):
                    W = torch.empty((M, N), device=dev)
                    assert m.dequant(e, kind, W.data_ptr(), s) == 0
                    off = [48, 48 + L.I * L.H * 3 // 8, 48 + 2 * L.I * L.H * 3 // 8][kind]
                    want = orc.dequant(L.records[e][off:], L.scales[e][kind], books[l], 3 * kind, M, N)
                    assert np.array_equal(bits(W.cpu().numpy()), bits(want)), (l, e, kind)
            cache.release(s)
            ops += [es.RELEASE]
            if look and l + 1 < n_layers:
                guess = look_d.cpu().numpy()[:look].tolist()
                cache.prefetch(l + 1, guess)
                ops += [es.PREFETCH, l + 1, len(guess)] + guess
            st = m.status(s)
            assert st == 0, (t, l, st)
            check_routing(orc, L, lg.cpu().numpy(), ids_d.cpu().numpy(), w_d.cpu().numpy())
            rc, ref = ols[l].apply(xs[l], ids_d.cpu().numpy(), w_d.cpu().numpy(), chunk=0)
            assert rc == 0
            e_ = rel_err(y.cpu().numpy(), ref)
            worst = max(worst, e_)
            assert e_ <= LAYER_RTOL, (t, l, e_)
    cache.sync()
    got = cache.stats()
    dry = warp_amd.ExpertCache(rec, n_slots * rec, policy=0, depth=depth, dry=True)
    _, dst = es.run_product(dry, ops)
    assert [got[k] for k in ("hits", "misses", "evictions", "prefetched", "spec_issued", "reads")] == dst
    say(f"  slots {n_slots}: hits {got['hits']} misses {got['misses']} evictions {got['evictions']} "
        f"spec {got['spec_issued']}, worst layer rel err {worst:.2e}")
    if n_slots < n_layers * 64:
        assert got["evictions"] > 0
    for m in ms:
        m.close()
    cache.close()


@pytest.mark.parametrize("n_slots,look", [(24, 6), (100, 0)])
def test_forward_cached(orc, n_slots, look):
    """The native cache path (one call per layer) against the oracle, and
    its cache decisions against a dry replay of the same calls."""
    say("test_forward_cached", n_slots, look)
    n_layers, T = 3, 8
    dev = torch.device("cuda:0")
    Ls = [dsv3_layer(l, 400 + l) for l in range(n_layers)]
    rec = Ls[0].rec_bytes
    host = torch.empty((n_layers * Ls[0].E, rec), dtype=torch.uint8, pin_memory=True)
    for l, L in enumerate(Ls):
        host[l * L.E:(l + 1) * L.E] = torch.from_numpy(
            np.frombuffer(L.bank(), np.uint8).reshape(L.E, rec).copy())
    cache = warp_amd.ExpertCache(rec, n_slots * rec, policy=0, depth=2)
    cache.set_source([host.data_ptr() + i * rec for i in range(n_layers * Ls[0].E)], n_layers, Ls[0].E)
    ms = [gpu_layer(L, records=False) for L in Ls]
    for m, L in zip(ms, Ls):
        assert m.bind_table([], [], codebook_id=L.cb_base) == 0
    ols = [orc.moe(L, 1) for L in Ls]
    s = stream()
    ops = []
    look_d = torch.empty((64,), dtype=torch.int32, device=dev)
    for t in range(T):
        for l, (L, m) in enumerate(zip(Ls, ms)):
            x = bf16_inputs(L, 1, 2000 * t + l)
            xd = torch.from_numpy(x).to(dev).to(torch.bfloat16)
            y = torch.full((1, L.H), float("nan"), device=dev)
            ids = torch.empty((1, 8), dtype=torch.int32, device=dev)
            w = torch.empty((1, 8), device=dev)
            nxt = ms[l + 1] if l + 1 < n_layers else None
            m.forward_cached(cache, l, xd.data_ptr(), y.data_ptr(), nxt=nxt, lookahead=look,
                             ids_ptr=ids.data_ptr(), w_ptr=w.data_ptr(), bf16=True, stream=s)
            assert m.status(s) == 0, (t, l)
            idh = ids.cpu().numpy()[0].tolist()
            ops += [es.HINT, l, 8] + idh
            for e in idh:
                ops += [es.HOLD, l, e]
            ops += [es.RELEASE]
            if nxt is not None and look:
                nxt.predict(xd.data_ptr(), look, look_d.data_ptr(), bf16=True, stream=s)
                g = look_d.cpu().numpy()[:look].tolist()
                ops += [es.PREFETCH, l + 1, len(g)] + g
            rc, ref = ols[l].apply(x, ids.cpu().numpy(), w.cpu().numpy(), chunk=0)
            assert rc == 0
            e_ = rel_err(y.cpu().numpy(), ref)
            assert e_ <= LAYER_RTOL, (t, l, e_)
    cache.sync()
    got = cache.stats()
    dry = warp_amd.ExpertCache(rec, n_slots * rec, policy=0, depth=2, dry=True)
    _, dst = es.run_product(dry, ops)
    assert [got[k] for k in ("hits", "misses", "evictions", "prefetched", "spec_issued", "reads")] == dst
    say(f"  hits {got['hits']} misses {got['misses']} spec {got['spec_issued']}")
    for m in ms:
        m.close()
    cache.close()


def test_get_slot_refill_waits_for_readers(orc):
    """A slot handed out by get() and let go by the policy before a release
    (the next two gets make it the victim) is refilled only after the work
    already enqueued on its stream: the layer reading it still sees the old
    record, bit for bit."""
    say("test_get_slot_refill_waits_for_readers")
    dev = torch.device("cuda:0")
    L = dsv3_layer(0, 500)
    rec = L.rec_bytes
    host = torch.empty((L.E, rec), dtype=torch.uint8, pin_memory=True)
    host[:] = torch.from_numpy(np.frombuffer(L.bank(), np.uint8).reshape(L.E, rec).copy())
    ref = gpu_layer(L)
    X = bf16_inputs(L, 1, 77)
    xd = torch.from_numpy(X).to(dev).to(torch.bfloat16)
    y0 = torch.empty((1, L.H), device=dev)
    ids0 = torch.empty((1, L.K), dtype=torch.int32, device=dev)
    ref.forward(xd.data_ptr(), 1, y0.data_ptr(), ids0.data_ptr(), None, None, bf16=True, stream=stream())
    assert ref.status(stream()) == 0
    ids = ids0.cpu().numpy()[0].tolist()
    # 9 slots: the 8 routed records, then one more get and a refill of the
    # first one's slot while the layer that reads it may still be queued
    cache = warp_amd.ExpertCache(rec, 9 * rec, policy=1, depth=0)
    cache.set_source([host.data_ptr() + e * rec for e in range(L.E)], 1, L.E)
    m = gpu_layer(L, records=False)
    s = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(s):
        sp = s.cuda_stream
        ptrs = [cache.get(0, e, sp) for e in ids]
        assert all(ptrs)
        assert m.bind_table(ids, ptrs, codebook_id=L.cb_base, stream=sp) == 0
        for _ in range(6):                           # a queue of readers
            y = torch.empty((1, L.H), device=dev)
            m.forward(xd.data_ptr(), 1, y.data_ptr(), None, None, None, bf16=True, stream=sp)
            outs.append(y)
        others = [e for e in range(L.E) if e not in ids][:2]
        for e in others:                             # LRU: the first slot goes
            assert cache.get(0, e, sp)
        assert any(cache.slot(0, e) < 0 for e in ids), "no routed record's slot was reused"
    torch.cuda.synchronize()
    assert m.status(stream()) == 0
    want = bits(y0.cpu().numpy())
    for y in outs:
        assert np.array_equal(bits(y.cpu().numpy()), want)
    cache.release(stream())
    m.close()
    ref.close()
    cache.close()


def _pinned_bank(Ls):
    rec = Ls[0].rec_bytes
    host = torch.empty((len(Ls) * Ls[0].E, rec), dtype=torch.uint8, pin_memory=True)
    for l, L in enumerate(Ls):
        host[l * L.E:(l + 1) * L.E] = torch.from_numpy(np.frombuffer(L.bank(), np.uint8).reshape(L.E, rec).copy())
    return host


def _run_cached(Ls, host, tokens, n_slots, depth, look, warm=None, save=None):
    """Every token through every layer by forward_cached: [(y, ids, w)]."""
    dev = torch.device("cuda:0")
    rec, E = Ls[0].rec_bytes, Ls[0].E
    cache = warp_amd.ExpertCache(rec, n_slots * rec, policy=0, depth=depth)
    cache.set_source([host.data_ptr() + i * rec for i in range(len(Ls) * E)], len(Ls), E)
    warmed = cache.warm(warm) if warm else 0
    ms = [gpu_layer(L, records=False) for L in Ls]
    for m, L in zip(ms, Ls):
        assert m.bind_table([], [], codebook_id=L.cb_base) == 0
    s = stream()
    outs = []
    for t in range(tokens):
        for l, (L, m) in enumerate(zip(Ls, ms)):
            xd = torch.from_numpy(bf16_inputs(L, 1, 7000 * t + l)).to(dev).to(torch.bfloat16)
            y = torch.full((1, L.H), float("nan"), device=dev)
            ids = torch.empty((1, L.K), dtype=torch.int32, device=dev)
            w = torch.empty((1, L.K), device=dev)
            nxt = ms[l + 1] if l + 1 < len(Ls) else None
            m.forward_cached(cache, l, xd.data_ptr(), y.data_ptr(), nxt=nxt, lookahead=look if nxt else 0,
                             ids_ptr=ids.data_ptr(), w_ptr=w.data_ptr(), bf16=True, stream=s)
            assert m.status(s) == 0, (t, l)
            outs.append((y.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()))
    cache.sync()
    st = cache.stats()
    if save:
        assert cache.save_usage(save, tokens) == 0
    for m in ms:
        m.close()
    cache.close()
    return outs, st, warmed


def test_cache_configs_bit_identical(orc, tmp_path):
    """Placement decides speed, never the numbers: the same tokens through
    layers holding their own records and through caches of every shape
    (everything resident, tight, read-ahead depth 0 and 2, lookahead 0
    and 6, warmed from a usage file) give bit-identical outputs, ids and
    weights."""
    say("test_cache_configs_bit_identical")
    n_layers, tokens = 3, 5
    Ls = [dsv3_layer(l, 800 + l) for l in range(n_layers)]
    dev = torch.device("cuda:0")
    base = []
    ms = [gpu_layer(L) for L in Ls]
    for t in range(tokens):
        for l, (L, m) in enumerate(zip(Ls, ms)):
            xd = torch.from_numpy(bf16_inputs(L, 1, 7000 * t + l)).to(dev).to(torch.bfloat16)
            y = torch.full((1, L.H), float("nan"), device=dev)
            ids = torch.empty((1, L.K), dtype=torch.int32, device=dev)
            w = torch.empty((1, L.K), device=dev)
            m.forward(xd.data_ptr(), 1, y.data_ptr(), ids.data_ptr(), w.data_ptr(), None, bf16=True, stream=stream())
            assert m.status(stream()) == 0
            base.append((y.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()))
    for m in ms:
        m.close()
    host = _pinned_bank(Ls)
    usage = str(tmp_path / "usage.waste")
    configs = [(n_layers * 64, 0, 0, None, usage), (24, 2, 6, None, None), (16, 0, 0, None, None),
               (16, 2, 6, None, None), (24, 2, 0, None, None), (24, 2, 6, usage, None)]
    for n_slots, depth, look, warm, save in configs:
        outs, st, warmed = _run_cached(Ls, host, tokens, n_slots, depth, look, warm=warm, save=save)
        say(f"  slots {n_slots} depth {depth} look {look} warm {warmed}: hits {st['hits']} misses {st['misses']}")
        if warm:
            assert warmed == 24
        for k, (a, b) in enumerate(zip(base, outs)):
            assert np.array_equal(a[1], b[1]), (n_slots, depth, look, k)
            assert np.array_equal(bits(a[0]), bits(b[0])) and np.array_equal(bits(a[2]), bits(b[2])), \
                (n_slots, depth, look, k)


def test_warm_fills_slots(orc, tmp_path):
    """A warmed cache's slots hold the records the usage file names before
    any demand: each slot, bound to a layer, passes the device header
    check and dequantises bit-exactly to the record's matrices."""
    say("test_warm_fills_slots")
    import struct
    Ls = [dsv3_layer(l, 820 + l) for l in range(2)]
    host = _pinned_bank(Ls)
    rec, E = Ls[0].rec_bytes, Ls[0].E
    path = str(tmp_path / "u.waste")
    picks = [(1, 5, 40), (0, 3, 30), (1, 63, 20), (0, 0, 10), (5, 1, 5)]     # (5, 1): not in the source
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQ", 0x47535557, 1, 9))
        for layer, e, hits in picks:
            f.write(struct.pack("<HHIII", layer, e, hits, 1, 0))
    cache = warp_amd.ExpertCache(rec, 8 * rec, policy=0, depth=0)
    cache.set_source([host.data_ptr() + i * rec for i in range(2 * E)], 2, E)
    assert cache.warm(path) == 4
    ms = [gpu_layer(L, records=False) for L in Ls]
    dev = torch.device("cuda:0")
    s = stream()
    for i, (layer, e, _) in enumerate(picks[:4]):
        assert cache.slot(layer, e) == i
        L, m = Ls[layer], ms[layer]
        p = cache.get(layer, e, s)
        assert p
        assert m.bind_table([e], [p], codebook_id=L.cb_base, stream=s) == 0
        books = orc.books(L.books_f16)[0]
        for kind, (M, N) in enumerate(L.shapes):
            W = torch.empty((M, N), device=dev)
            assert m.dequant(e, kind, W.data_ptr(), s) == 0
            off = [48, 48 + L.I * L.H * 3 // 8, 48 + 2 * L.I * L.H * 3 // 8][kind]
            want = orc.dequant(L.records[e][off:], L.scales[e][kind], books, 3 * kind, M, N)
            assert np.array_equal(bits(W.cpu().numpy()), bits(want)), (layer, e, kind)
        assert m.status(s) == 0
        cache.release(s)
    st = cache.stats()
    assert st["hits"] == 4 and st["misses"] == 0 and st["reads"] == 0
    for m in ms:
        m.close()
    cache.close()
