# SPDX-License-Identifier: Apache-2.0
"""The expert cache: the restatement of src/ecache.c pinned against the
engine's own ecache.c (compiled from its sources into oracle/_ref) and
against closed-form cases, then the product cache's decisions against the
restatement, slot for slot, on the reference's routing traces
(tests/trace_olmoe_299.jsonl and tests/trace_kimi_300.jsonl there).

CPU only: the product runs with dry=1 (its policy, no device).  The device
side (fills, stream order) is tests/test_gpu_ecache.py.
"""
import os

import numpy as np
import pytest

import ecache_script as es
from oracle_lib import REF_SO, Oracle, Ref, fp, ptr

REC = 4096


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    return Ref()


@pytest.fixture(scope="module")
def traces():
    return {n: es.load_trace(n) for n in ("trace_olmoe_299", "trace_kimi_300")}


def product(n_slots, depth, policy):
    import warp_amd
    return warp_amd.ExpertCache(REC, n_slots * REC, policy=policy, depth=depth, dry=True)


# ---- the restatement against the engine's own cache ----------------------

CASES = [  # (name, tokens, script kwargs, depth)
    ("sync-get", 40, dict(hold=False, hint=False), 0),
    ("hint-hold", 40, dict(hold=True, hint=True), 2),
    ("hint-hold-lookahead", 40, dict(hold=True, hint=True, lookahead=6), 2),
    ("hint-get-lookahead", 40, dict(hold=False, hint=True, lookahead=6), 2),
    ("deep-lookahead", 30, dict(hold=True, hint=True, lookahead=16), 8),
    ("admit-then-hold", 30, dict(hold=True, hint=True, admit_first=40), 2),
]


@pytest.mark.parametrize("trace", ["trace_olmoe_299", "trace_kimi_300"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("n_slots", [25, 100, 201, 402, 1000])
@pytest.mark.parametrize("policy", [0, 1], ids=["lfru", "lru"])
def test_oracle_matches_engine_cache(orc, ref, traces, trace, case, n_slots, policy):
    """Every slot the engine's cache hands out, and every counter, equal."""
    _, ntok, kw, depth = case
    ops = es.layer_calls(traces[trace][:ntok], **kw)
    r_out, r_st = ref.ecache_run(ops, n_slots, depth, policy)
    o_out, o_st = orc.ecache_run(ops, n_slots, depth, policy)
    assert o_st == r_st
    assert o_out == r_out


def test_oracle_matches_engine_cache_full_traces(orc, ref, traces):
    for name, tr in traces.items():
        ops = es.layer_calls(tr, hold=True, hint=True, lookahead=6)
        n = {"trace_olmoe_299": 300, "trace_kimi_300": 1600}[name]
        r = ref.ecache_run(ops, n, 2, 0)
        o = orc.ecache_run(ops, n, 2, 0)
        assert o == r, name


# ---- closed forms -----------------------------------------------------------

def test_no_slots_every_access_misses(orc, traces):
    ops = es.demand_only(traces["trace_olmoe_299"][:20])
    out, st = orc.ecache_run(ops, 0, 0, 0)
    n = len(ops) // 3
    assert st[:3] == [0, n, 0] and st[5] == n
    assert out == [-1] * n


@pytest.mark.parametrize("trace", ["trace_olmoe_299", "trace_kimi_300"])
def test_cache_that_holds_everything_misses_each_record_once(orc, trace, traces):
    tr = traces[trace]
    keys = [(L, e) for layers in tr for L, ids in enumerate(layers) for e in ids]
    distinct = len(set(keys))
    ops = es.demand_only(tr)
    for policy in (0, 1):
        out, st = orc.ecache_run(ops, len(tr[0]) * 256, 0, policy)
        assert st[1] == distinct and st[0] == len(keys) - distinct and st[2] == 0
        # slots fill in first-touch order and a record never moves
        first = {}
        for k, s in zip(keys, out):
            first.setdefault(k, s)
            assert first[k] == s
        assert sorted(set(out)) == list(range(distinct))


def test_below_one_tokens_working_set_nothing_hits(orc, traces):
    """src/ecache.h:232-234: a cache smaller than one token's working set
    (16 layers x 8 = 128 records here) gets no hits from the demand stream,
    the fraction measured on the engine."""
    ops = es.demand_only(traces["trace_olmoe_299"])
    for n in (8, 32, 61):
        out, st = orc.ecache_run(ops, n, 0, 0)
        assert st[0] == 0, n


def test_lfru_keeps_the_frequent_record_lru_the_recent_one(orc):
    """Three slots, A A A B C D A.  For D the last record handed out (C) is
    pinned, so the choice is A (3 hits, older) or B (1 hit, newer): LFRU
    evicts B and the last A hits; LRU evicts A and it misses."""
    A, B, Cc, D = (0, 1), (0, 2), (0, 3), (0, 4)
    ops = []
    for k in (A, A, A, B, Cc, D, A):
        ops += [es.GET, k[0], k[1]]
    _, st = orc.ecache_run(ops, 3, 0, 0)
    assert st[:2] == [3, 4]
    _, st = orc.ecache_run(ops, 3, 0, 1)
    assert st[:2] == [2, 5]


def test_hint_reads_are_misses_not_later_hits(orc):
    """A hinted record is a miss when its read is issued; the get that then
    finds it is not a hit (src/ecache.c fresh); the next one is."""
    ops = [es.HINT, 0, 2, 5, 9, es.GET, 0, 5, es.GET, 0, 9, es.GET, 0, 5]
    _, st = orc.ecache_run(ops, 16, 2, 0)
    hits, misses, ev, prefetched, spec, reads = st
    assert (hits, misses, prefetched, reads) == (1, 2, 2, 2)


def test_lookahead_reads_count_bytes_not_misses(orc):
    ops = [es.PREFETCH, 1, 3, 4, 5, 6, es.GET, 1, 4, es.GET, 1, 7]
    _, st = orc.ecache_run(ops, 16, 2, 0)
    hits, misses, ev, prefetched, spec, reads = st
    assert (hits, misses, spec, reads) == (1, 1, 3, 4)


def test_sync_cache_ignores_hints_and_lookahead(orc):
    ops = [es.HINT, 0, 2, 5, 9, es.PREFETCH, 0, 1, 7, es.ADMIT, 0, 3]
    out, st = orc.ecache_run(ops, 16, 0, 0)
    assert out == [0] and st == [0, 0, 0, 0, 0, 0]


def test_predict_next_is_a_stable_argsort(orc):
    """predict_next_moe: top n of score + bias, ties to the lower id."""
    rng = np.random.default_rng(3)
    for sf in (0, 1, 2):
        lg = rng.standard_normal(256).astype(np.float32)
        lg[17] = lg[40] = lg[200] = 1.25                   # a three-way tie
        bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
        bias[17] = bias[40] = bias[200] = 0.5
        sc = np.zeros(256, np.float32)
        orc.lib.orc_router_scores(sf, ptr(lg, fp), ptr(sc, fp), 256)
        p = (sc + bias).astype(np.float32)
        want = np.argsort(-p, kind="stable")[:16]
        got = orc.predict_next(sf, lg, bias, 16)
        assert list(got) == list(want)
        assert list(orc.predict_next(sf, lg, None, 5)) == list(np.argsort(-sc, kind="stable")[:5])


# ---- the product cache against the restatement ------------------------------

@pytest.mark.parametrize("trace", ["trace_olmoe_299", "trace_kimi_300"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("n_slots", [0, 25, 201, 1000])
@pytest.mark.parametrize("policy", [0, 1], ids=["lfru", "lru"])
def test_product_decisions_equal_oracle(orc, traces, trace, case, n_slots, policy):
    _, ntok, kw, depth = case
    ops = es.layer_calls(traces[trace][:ntok], **kw)
    o_out, o_st = orc.ecache_run(ops, n_slots, depth, policy)
    c = product(n_slots, depth, policy)
    p_out, p_st = es.run_product(c, ops)
    assert p_st == o_st
    assert p_out == o_out


def test_product_full_traces_and_residency(orc, traces):
    for name, tr in traces.items():
        ops = es.layer_calls(tr, hold=True, hint=True, lookahead=6)
        n_layers = len(tr[0])
        # residency asked before every 50th hold
        masks = {}
        w = 0
        k = 0
        while w < len(ops):
            op = ops[w]
            if op == es.HOLD:
                if k % 50 == 0:
                    masks[w] = (ops[w + 1], 256)
                k += 1
                w += 3
            elif op == es.RELEASE:
                w += 1
            elif op in (es.GET, es.ADMIT):
                w += 3
            else:
                w += 3 + ops[w + 2]
        n = 64 * n_layers
        o = orc.ecache_run(ops, n, 2, 0, masks=masks)
        c = product(n, 2, 0)
        p = es.run_product(c, ops, masks=masks)
        assert p[0] == o[0] and p[1] == o[1], name
        for w in masks:
            assert list(p[2][w]) == list(o[2][w]), (name, w)
        hit_rate = o[1][0] / (o[1][0] + o[1][1])
        assert 0.0 < hit_rate < 1.0


def test_product_hold_limit_and_release(orc):
    c = product(200, 0, 0)
    ptrs = [c.hold(0, e) for e in range(64)]
    assert all(ptrs)
    assert not c.hold(0, 64)                 # the held set is full
    c.release()
    assert c.hold(0, 64)


def test_product_rejects_bad_arguments():
    import warp_amd
    with pytest.raises(warp_amd.HipError):
        warp_amd.ExpertCache(1000, 10 * 1000, dry=True)      # not a multiple of 256
    with pytest.raises(warp_amd.HipError):
        warp_amd.ExpertCache(REC, 10 * REC, policy=2, dry=True)
    with pytest.raises(warp_amd.HipError):
        warp_amd.ExpertCache(REC, 10 * REC, depth=-1, dry=True)


# ---- the learned hotlist (usage.waste) ----------------------------------

def _usage(path, entries, magic=0x47535557, tokens=7):
    import struct
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQ", magic, 1, tokens))
        for layer, e, hits, last in entries:
            f.write(struct.pack("<HHIII", layer, e, hits, last, 0))


@pytest.mark.parametrize("trace", ["trace_olmoe_299", "trace_kimi_300"])
@pytest.mark.parametrize("n_slots,depth,policy", [(100, 0, 0), (201, 2, 0), (402, 2, 1), (25, 2, 0)])
def test_usage_save_and_warm_equal_engine(ref, traces, tmp_path, trace, n_slots, depth, policy):
    """save_usage writes the engine's file byte for byte after the same
    script; a cache warmed from it then decides as the engine's warmed
    cache does, slot for slot (src/ecache.c:827-913)."""
    tr = traces[trace]
    kw = dict(hold=True, hint=depth > 0, lookahead=6 if depth else 0)
    a, b = str(tmp_path / "engine.waste"), str(tmp_path / "product.waste")
    ref.ecache_run(es.layer_calls(tr[:40], **kw), n_slots, depth, policy, save=a)
    c = product(n_slots, depth, policy)
    es.run_product(c, es.layer_calls(tr[:40], **kw))
    raw = open(a, "rb").read()
    tokens = int(np.frombuffer(raw[8:16], np.uint64)[0])
    assert c.save_usage(b, tokens) == 0
    assert open(b, "rb").read() == raw
    assert (len(raw) - 16) // 16 > 0
    ops2 = es.layer_calls(tr[40:90], **kw)
    r_out, r_st = ref.ecache_run(ops2, n_slots, depth, policy, warm=a)
    r_warm = ref.ecache_warmed()
    c2 = product(n_slots, depth, policy)
    assert c2.warm(a) == r_warm == min(n_slots, (len(raw) - 16) // 16)
    p_out, p_st = es.run_product(c2, ops2)
    assert p_st == r_st
    assert p_out == r_out


def test_warm_order_and_limits(tmp_path):
    """Hottest first, ties by (layer, expert); the engine walks the first
    min(entries, slots) entries of the sorted file, so a duplicate or a
    resident record uses up a place (src/ecache.c:890-910)."""
    path = str(tmp_path / "u.waste")
    ents = [(0, 5, 3, 1), (1, 2, 9, 2), (0, 1, 9, 3), (2, 7, 1, 4), (0, 1, 9, 5), (1, 0, 3, 6)]
    _usage(path, ents)
    c = product(3, 0, 0)
    # sorted: (0,1) (0,1) (1,2) | (0,5) (1,0) (2,7); three places, one a duplicate
    assert c.warm(path) == 2
    assert [c.slot(0, 1), c.slot(1, 2)] == [0, 1]
    assert c.slot(0, 5) == -1 and c.slot(1, 0) == -1
    assert c.stats()["reads"] == 0 and c.stats()["misses"] == 0
    # a warmed record is a hit on its first demand
    c.get(0, 1)
    assert c.stats()["hits"] == 1
    four = product(4, 0, 0)
    assert four.warm(path) == 3 and four.slot(0, 5) == 2 and four.slot(1, 0) == -1
    big = product(10, 0, 0)
    assert big.warm(path) == 5
    assert big.warm(path) == 0                       # all resident already


def test_warm_skips_records_the_source_lacks(tmp_path):
    path = str(tmp_path / "u.waste")
    _usage(path, [(0, 1, 5, 1), (3, 0, 4, 2), (1, 9, 3, 3), (1, 2, 2, 4)])
    c = product(8, 0, 0)
    c.set_source([4096 * (k + 1) for k in range(2 * 4)], 2, 4)     # layers 0-1, experts 0-3
    assert c.warm(path) == 2
    assert c.slot(0, 1) == 0 and c.slot(1, 2) == 1
    assert c.slot(3, 0) == -1 and c.slot(1, 9) == -1


def test_warm_refusals(tmp_path):
    import warp_amd
    c = product(4, 0, 0)
    assert c.warm(str(tmp_path / "missing.waste")) == warp_amd.EIO
    bad = str(tmp_path / "bad.waste")
    _usage(bad, [(0, 1, 1, 1)], magic=0x12345678)
    assert c.warm(bad) == warp_amd.EFORMAT
    empty = str(tmp_path / "empty.waste")
    _usage(empty, [])
    assert c.warm(empty) == 0
    with open(empty, "ab") as f:
        f.write(b"\0" * 7)                         # a partial entry is ignored
    assert c.warm(empty) == 0
    assert c.save_usage(str(tmp_path / "no_dir" / "u.waste"), 0) == warp_amd.EIO
    z = product(0, 0, 0)
    assert z.warm(bad) == 0                         # no slots: nothing to do


def test_lookahead_use_and_waste_counted():
    """What became of the lookahead reads: demanded while resident (used)
    or evicted first (wasted); counters only, the decisions unchanged (a
    dry cache of 4 slots)."""
    import warp_amd
    rb = 4096
    c = warp_amd.ExpertCache(rb, 4 * rb, policy=0, depth=2, dry=True)
    c.prefetch(1, [4, 5])                      # two lookahead reads
    assert c.get(1, 4)                         # one demanded: used
    st = c.stats()
    assert (st["spec_issued"], st["spec_used"], st["spec_wasted"]) == (2, 1, 0)
    assert c.get(1, 4)                         # a second demand counts once
    for e in (10, 11, 12, 13, 14, 15):         # misses push every older record out
        assert c.get(2, e)
    st = c.stats()
    assert (st["spec_used"], st["spec_wasted"]) == (1, 1)   # expert 5 left unread
    assert st["spec_issued"] == 2 and st["hits"] == 2 and st["misses"] == 6
    c.close()
