# SPDX-License-Identifier: Apache-2.0
"""The many-token path (moe_chunk, src/model.c:7110-7285, as grouped
products on the matrix cores) against the oracle.

Bars: router logits max relative error 1e-5 (fp32 products); expert ids and
weights bit-exact against the oracle's router on the device's logits; layer
output max relative error 1e-3, normwise, against the oracle's moe_chunk on
the same routing (fp16 operands, fp32 accumulation).
"""
import sys

import numpy as np
import pytest

from gpu_util import LAYER_RTOL, LOGIT_RTOL, gpu_layer, rel_err, run_forward
from oracle_lib import Oracle

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402
from test_gpu_parity import check_routing, make_case  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


def check_layer(orc, L, X, bf16, y, ids, w, lg, tag):
    ol = orc.moe(L, 1)
    e_lg = rel_err(lg, ol.logits(X))
    assert e_lg <= LOGIT_RTOL, (tag, e_lg)
    check_routing(orc, L, lg, ids, w)
    rc, ref = ol.apply(X, ids, w, chunk=1)
    assert rc == 0
    e = rel_err(y, ref)
    say(f"  {tag}: logits rel err {e_lg:.2e}, layer rel err {e:.3e}, distinct experts "
        f"{len(np.unique(ids))}")
    assert e <= LAYER_RTOL


@pytest.mark.parametrize("name,T", [("olmoe_small", 48), ("kimi_small", 40), ("dsv3_small", 64),
                                    ("dsv3_small", 200)])
def test_prefill_parity(orc, name, T):
    say("test_prefill_parity", name, T)
    L, X, bf16 = make_case(name, T)
    m = gpu_layer(L, max_tokens=T, prefill_min=16)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16)
    m.close()
    assert st == 0
    check_layer(orc, L, X, bf16, y, ids, w, lg, f"{name} T={T}")


def test_prefill_long_segments(orc):
    """A bias that puts two experts in each of four groups ahead of all
    others: those groups win the group stage and the eight experts take
    every token, so their segments span several 128-row blocks of the
    grouped products."""
    say("test_prefill_long_segments")
    L, X, bf16 = make_case("dsv3_small", 300)
    gs = L.E // L.n_group
    hot = np.array([g * gs + o for g in (0, 2, 5, 7) for o in (1, 6)])
    L.bias = L.bias.copy()
    L.bias[hot] += 5.0
    m = gpu_layer(L, max_tokens=300, prefill_min=16)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16)
    m.close()
    assert st == 0
    assert set(np.unique(ids)) == set(hot.tolist())
    check_layer(orc, L, X, bf16, y, ids, w, lg, "dsv3_small T=300, 8 hot experts")


def test_prefill_matches_decode_path(orc):
    """The same tokens through both paths of one layer agree within the bar
    (different arithmetic, same routing)."""
    say("test_prefill_matches_decode_path")
    L, X, bf16 = make_case("kimi_small", 24)
    m1 = gpu_layer(L, max_tokens=24, prefill_min=32)      # decode kernels
    m2 = gpu_layer(L, max_tokens=24, prefill_min=8)       # matrix cores
    st1, y1, ids1, w1, _ = run_forward(torch, m1, L, X, bf16)
    st2, y2, ids2, w2, _ = run_forward(torch, m2, L, X, bf16)
    m1.close()
    m2.close()
    assert st1 == 0 and st2 == 0
    assert np.array_equal(ids1, ids2)
    e = rel_err(y2, y1)
    say(f"  prefill vs decode kernels: rel err {e:.3e}")
    assert e <= LAYER_RTOL


def test_prefill_unbound_expert(orc):
    """A routed expert without a record: status reports it, its pairs add
    nothing, and the rest of the layer is unaffected."""
    say("test_prefill_unbound_expert")
    L, X, bf16 = make_case("dsv3_small", 64)
    m = gpu_layer(L, max_tokens=64, prefill_min=16)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16)
    assert st == 0
    gone = int(np.bincount(ids.reshape(-1)).argmax())
    assert m.bind_expert(gone, 0, L.rec_bytes) == 0
    st2, y2, ids2, w2, _ = run_forward(torch, m, L, X, bf16)
    m.close()
    assert st2 == warp_amd.EUNBOUND
    assert np.array_equal(ids, ids2)
    ol = orc.moe(L, 1)
    w_masked = np.where(ids == gone, 0.0, w).astype(np.float32)
    rc, ref = ol.apply(X, ids, w_masked, chunk=1)
    assert rc == 0
    assert rel_err(y2, ref) <= LAYER_RTOL


def test_prefill_out_of_fp16_range(orc):
    """Tokens whose activations (2^17 x N(0,1): beyond 65504) or SwiGLU
    outputs (2^11 x N(0,1) inputs) leave fp16's range: the chunk runs again
    on the fp32 decode kernels with the routing it has, so the status is
    clean and every output matches the oracle's moe_chunk."""
    say("test_prefill_out_of_fp16_range")
    L, X, bf16 = make_case("dsv3_small", 64)
    X = X.copy()
    X[[3, 40]] *= np.float32(2.0 ** 11)
    X[17] *= np.float32(2.0 ** 17)
    m = gpu_layer(L, max_tokens=64, prefill_min=16)
    st, y, ids, w, lg = run_forward(torch, m, L, X, bf16)
    m.close()
    assert st == 0, warp_amd.ERRORS.get(st, st)
    assert float(np.abs(X).max()) > 65504.0
    check_layer(orc, L, X, bf16, y, ids, w, lg, "dsv3_small T=64, tokens out of fp16 range")
