# SPDX-License-Identifier: Apache-2.0
"""The expert-cache stack's synthetic routing (bench.stack_inputs) on the
CPU: planted tokens look like N(0,1) noise, their router logits carry the
stated popularity, reuse and lookahead overlap, and the Zipf fit used to
report them recovers a known exponent.  Selections go through the oracle's
group-limited router (sigmoid, 8 groups / 4 kept, top-8)."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import bench  # noqa: E402
from oracle_lib import Oracle  # noqa: E402

torch = pytest.importorskip("torch")
E, H, K, T = 256, 2048, 8, 200


def routers(n, seed=3):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal((E, H), np.float32) * 0.02).astype(np.float32) for _ in range(n)]


def select(orc, logits):
    bias = np.zeros(E, np.float32)
    out = []
    for row in logits:
        rc, idx, _, _ = orc.route(row.astype(np.float32), bias, E, K, 0, 1, 2.5, 8, 4)
        assert rc == K
        out.append(set(idx.tolist()))
    return out


def test_zipf_mle_recovers_exponent():
    r = np.arange(1, 257, dtype=np.float64)
    for s in (0.8, 1.1, 1.5):
        assert abs(bench.zipf_mle(np.round(1e7 * r ** -s)) - s) < 0.003


def test_sticky_gumbel_keeps_its_share():
    g = bench.sticky_gumbel(np.random.default_rng(0), 4000, 256, 0.63)
    same = (g[1:] == g[:-1]).mean()
    assert abs(same - 0.63) < 0.005
    # every row is Gumbel (mean 0.5772, variance pi^2/6); a value lasts
    # about 2.7 rows, so the sample is worth about a quarter of its size
    assert abs(g.mean() - 0.5772) < 0.012 and abs(g.var() - np.pi ** 2 / 6) < 0.04


def test_planted_tokens():
    orc = Oracle()
    W = routers(3)
    X, ranks = bench.stack_inputs(torch, W, T, 1.1, 0.63, 0.88, 0.5, seed=11, device="cpu")
    Xf = X.float().numpy()
    assert X.shape == (T, 3, H)
    assert abs(Xf.std() - 1.0) < 0.05 and abs(Xf.mean()) < 0.02          # N(0,1)-like
    sel = [select(orc, Xf[:, L] @ W[L].T) for L in range(3)]
    reuse = np.mean([len(s[t] & s[t - 1]) / K for s in sel for t in range(1, T)])
    assert 0.55 < reuse < 0.65
    distinct = np.mean([len(set().union(*s)) for s in sel])
    assert 150 < distinct < 190                # the generator's ~168 at 200 tokens
    # popular ranks are picked more: rank-1 expert in most tokens, the tail rarely
    by_rank = np.zeros(E)
    for L in range(3):
        for S in sel[L]:
            np.add.at(by_rank, ranks[L][np.array(sorted(S))], 1)
    assert by_rank[0] > 0.7 * T * 3 and by_rank[:128].sum() > 4 * by_rank[128:].sum()
    # the lookahead: the next layer's router on this layer's token
    prec = []
    for L in range(2):
        sc = Xf[:, L] @ W[L + 1].T
        for t in range(T):
            g = np.argsort(-sc[t], kind="stable")[:6]
            prec.append(len(sel[L + 1][t] & set(g.tolist())) / 6)
    assert 0.74 < np.mean(prec) < 0.88        # about the engine's measured 81%


def test_full_overlap_is_full_reuse():
    orc = Oracle()
    W = routers(2, seed=5)
    X, _ = bench.stack_inputs(torch, W, 20, 1.1, 1.0, 1.0, 0.5, seed=2, device="cpu")
    Xf = X.float().numpy()
    s0 = select(orc, Xf[:, 0] @ W[0].T)
    assert all(s0[t] == s0[0] for t in range(20))
    # identical noise in the next layer's planted logits: same top-8
    s1 = select(orc, Xf[:, 1] @ W[1].T)
    look = select(orc, Xf[:, 0] @ W[1].T)
    assert np.mean([len(a & b) for a, b in zip(s1, look)]) > 7.5


def test_group_top_is_the_group_limited_route():
    """bench.group_top: the oracle's group-limited route (8 groups, 4 kept,
    no bias) on the same sigmoid scores, in its order."""
    orc = Oracle()
    rng = np.random.default_rng(5)
    for _ in range(50):
        lg = rng.standard_normal(256).astype(np.float32)
        sc = orc.router_scores(0, lg)
        for n in (1, 6, 8, 64):
            rc, want, _, _ = orc.route(lg, None, 256, n, 0, 0, 1.0, 8, 4)
            assert rc == n
            assert list(bench.group_top(sc.astype(np.float64), n, 8, 4)) == list(want)
