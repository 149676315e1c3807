# SPDX-License-Identifier: Apache-2.0
"""The persistent decode mode (decode.hip, set_decode(1)) against the
oracle and the staged kernels, on the benchmark shapes.

Bars: ids and weights bit-exact against the oracle's routing of the
launch's own logits; logits within 1e-5 of the oracle's router; layer
output within 1e-3 (normwise) of the oracle's layer on that routing; the
staged path on the same token picks the same experts and lands within
1e-3 of the one-launch output.  Repeated launches check that every launch
leaves its stage counters zero for the next one; an unbound expert is
reported and the next launch is clean.
"""
import sys

import numpy as np
import pytest

from gpu_util import LAYER_RTOL, rel_err
from test_gpu_fullsize import FullLayer, check_layer

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from oracle_lib import Oracle
    return Oracle()


@pytest.mark.parametrize("name", ["olmoe", "kimi", "dsv3"])
def test_decode1_parity(orc, name):
    say("test_decode1_parity", name)
    L = FullLayer(name, 1)
    try:
        for seed in range(3):
            x = L.tokens(1, seed=2000 + seed)
            L.m.set_decode(1)
            ids1 = check_layer(orc, L, x, chunk=False)
            st1, y1, i1, w1, _ = L.forward(x)
            assert st1 == 0 and np.array_equal(i1, ids1)
            L.m.set_decode(0)
            st0, y0, i0, w0, _ = L.forward(x)
            assert st0 == 0
            assert np.array_equal(i0, i1), (i0, i1)
            e = rel_err(y1, y0)
            say(f"  seed {seed}: one-launch vs staged rel err {e:.3e}")
            assert e <= LAYER_RTOL
    finally:
        L.close()


def test_decode1_repeated(orc):
    """Many launches in a row, each on a fresh token, interleaved with staged
    forwards: every one agrees with the staged kernels."""
    say("test_decode1_repeated")
    L = FullLayer("dsv3", 1)
    try:
        for i in range(24):
            x = L.tokens(1, seed=3000 + i)
            L.m.set_decode(1)
            st1, y1, i1, w1, _ = L.forward(x)
            assert st1 == 0, (i, st1)
            if i % 3 == 0:
                L.m.set_decode(0)
                st0, y0, i0, w0, _ = L.forward(x)
                assert st0 == 0 and np.array_equal(i0, i1)
                assert rel_err(y1, y0) <= LAYER_RTOL
            else:
                assert np.isfinite(y1).all() and np.abs(y1).max() > 0
    finally:
        L.close()


def test_decode1_unbound_then_clean(orc):
    """An unrouted-to expert may be unbound; a routed one is reported, and
    the launch after it (the expert bound again) is clean and correct."""
    say("test_decode1_unbound_then_clean")
    L = FullLayer("kimi", 1)
    L.m.set_decode(1)
    try:
        x = L.tokens(1, seed=4000)
        st, y, ids, w, _ = L.forward(x)
        assert st == 0
        e = int(ids[0, 3])
        assert L.m.bind_expert(e, 0, L.rb) == 0           # NULL unbinds
        st, *_ = L.forward(x)
        assert st == warp_amd.EUNBOUND, st
        assert L.m.bind_expert(e, L.slab.data_ptr() + e * L.rb, L.rb) == 0
        check_layer(orc, L, x, chunk=False)
    finally:
        L.close()
