# SPDX-License-Identifier: Apache-2.0
"""Cache scripts: the calls moe_layer makes on its expert cache, as a flat
list of ints that the restatement, the engine's own ecache.c (through
oracle/_ref) and the product library can each replay.

Words: 0 L e get | 1 L e hold | 2 release | 3 L n ids.. hint |
4 L n ids.. prefetch | 5 L e admit.
"""
import json
import os

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GET, HOLD, RELEASE, HINT, PREFETCH, ADMIT = range(6)


def load_trace(name):
    """[token][layer] -> sorted expert ids (the engine's routing dumps,
    tests/trace_*.jsonl in the reference)."""
    with open(os.path.join(GOLDEN, name + ".jsonl")) as f:
        return [json.loads(line)["layers"] for line in f]


def layer_calls(trace, *, hold=True, hint=True, lookahead=0, admit_first=0):
    """moe_layer's sequence per layer (src/model.c:5639-5700, 5926-5930):
    hint the layer's ids, hold each, release, then the lookahead's guess
    for the next layer.  The guess here is the previous token's set at the
    next layer, cut to `lookahead` (a stand-in for the router lookahead,
    which needs the hidden state).  admit_first: admit that many records
    of layer 0 before the first token (the background fill)."""
    ops = []
    for e in range(admit_first):
        ops += [ADMIT, 0, e]
    for t, layers in enumerate(trace):
        for L, ids in enumerate(layers):
            if hint:
                ops += [HINT, L, len(ids)] + list(ids)
            for e in ids:
                ops += [HOLD if hold else GET, L, e]
            ops += [RELEASE]
            if lookahead and t > 0 and L + 1 < len(layers):
                g = list(trace[t - 1][L + 1][:lookahead])
                ops += [PREFETCH, L + 1, len(g)] + g
    return ops


def demand_only(trace):
    """Every (layer, expert) of every token once, in layer order, through
    get(): the plain demand stream."""
    ops = []
    for layers in trace:
        for L, ids in enumerate(layers):
            for e in ids:
                ops += [GET, L, e]
    return ops


def run_product(cache, ops, masks=None):
    """Replays ops on a warp_amd.ExpertCache (dry): (outputs, stats list
    in the restatement's order, masks)."""
    out, got = [], {}
    w = 0
    rb = cache.rec_bytes
    while w < len(ops):
        if masks and w in masks:
            layer, n = masks[w]
            got[w] = cache.resident_mask(layer, n)
        op = ops[w]
        if op in (GET, HOLD):
            p = (cache.get if op == GET else cache.hold)(ops[w + 1], ops[w + 2])
            out.append(-1 if not p else p // rb - 1)
            w += 3
        elif op == ADMIT:
            out.append(cache.admit(ops[w + 1], ops[w + 2]))
            w += 3
        elif op == RELEASE:
            cache.release()
            w += 1
        else:
            n = ops[w + 2]
            ids = ops[w + 3:w + 3 + n]
            (cache.hint if op == HINT else cache.prefetch)(ops[w + 1], ids)
            w += 3 + n
    s = cache.stats()
    st = [s["hits"], s["misses"], s["evictions"], s["prefetched"], s["spec_issued"], s["reads"]]
    return (out, st, got) if masks else (out, st)
