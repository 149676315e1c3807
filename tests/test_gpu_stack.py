# SPDX-License-Identifier: Apache-2.0
"""The expert-cache stack as bench.py measures it, on an MI355X.

bench.stack_setup builds what the bench's `expert_cache` line runs: 58
DeepSeek-V3-shaped layers (256 experts of 16.5 MB VQ3R records, the 4-bit
shared expert, each layer its own router), the 4.2 GB host bank in pinned
memory, an HBM cache of 64 GB of slots filled by hipMemcpyAsync, and tokens
whose routing follows Zipf(1.1) popularity with 0.6 token-to-token reuse
and the engine's lookahead quality.  Ten tokens decode through all 58 layers
with the lookahead on (moe_layer's cache path, src/model.c:5639-5700,
5921-5930).  For a sample of (token, layer) pairs, each token's last layer
and layers 0, 14, 29 and 43: the ids and weights are bit-exact against the
oracle's routing on the device's logits, and the layer output is within
1e-3 of the oracle's layer on the same records.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from gpu_util import LAYER_RTOL, rel_err
from oracle_lib import Oracle, OrcMoe, fp, ptr, u8p

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402
from warp_amd import synth  # noqa: E402
from test_gpu_fullsize import _ot, bits  # noqa: E402

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


def test_stack_measured_scale(orc):
    say("test_stack_measured_scale")
    cfg = synth.CONFIGS["dsv3"]
    H, E, K, I = cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]
    T, NL, look = 10, 58, 6
    dev = torch.device("cuda:0")
    books = synth.codebooks(0, H, I)
    layers, routers, cache, host, X, _, rb = bench.stack_setup(torch, warp_amd, synth, cfg, books, T, NL)
    say(f"  {NL} layers, {cache.n_slots} slots of {rb} B")
    Y = torch.full((T, NL, H), float("nan"), dtype=torch.float32, device=dev)
    ids = torch.empty((T, NL, K), dtype=torch.int32, device=dev)
    w = torch.empty((T, NL, K), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    esz = X.element_size()

    def xp(t, L):
        return X.data_ptr() + (t * NL + L) * H * esz

    for t in range(T):
        for L in range(NL):
            nxt = layers[L + 1] if L + 1 < NL else None
            layers[L].forward_cached(cache, L, xp(t, L), Y[t, L].data_ptr(), nxt=nxt,
                                     lookahead=look if nxt else 0, ids_ptr=ids[t, L].data_ptr(),
                                     w_ptr=w[t, L].data_ptr(), bf16=True, stream=s)
    torch.cuda.synchronize()
    cache.sync()
    for L, m in enumerate(layers):
        assert m.status(s) == 0, L
    st = cache.stats()
    say(f"  hits {st['hits']} misses {st['misses']} evictions {st['evictions']} lookahead reads "
        f"{st['spec_issued']}")
    assert st["misses"] > 0 and st["hits"] > 0
    # the sampled layers' logits, recomputed by route() (no cache access)
    sample = [(t, L) for t in range(T) for L in sorted({0, 14, 29, 43, NL - 1})]
    lg = torch.empty((len(sample), E), dtype=torch.float32, device=dev)
    sid = torch.empty((K,), dtype=torch.int32, device=dev)
    sw = torch.empty((K,), dtype=torch.float32, device=dev)
    for i, (t, L) in enumerate(sample):
        layers[L].route(xp(t, L), 1, sid.data_ptr(), sw.data_ptr(), lg[i].data_ptr(), bf16=True, stream=s)
    torch.cuda.synchronize()
    lgh, idh, wh, yh = lg.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), Y.cpu().numpy()
    xh = X.to(torch.float32).cpu().numpy()
    # the oracle's layers: the host bank's records (every layer reads the same
    # 256 records), each layer's router, a zero bias, the shared expert
    _, bT = orc.books(books)
    _, _, sh = synth.trunk(cfg, 1)
    bias = np.zeros(E, np.float32)
    recs = (u8p * E)(*[C.cast(host.data_ptr() + e * rb, u8p) for e in range(E)])
    rts = {L: synth.Tensor.make(cfg["router_fmt"], routers[L]) for L in {L for _, L in sample}}
    worst = 0.0
    for i, (t, L) in enumerate(sample):
        om = OrcMoe(H, E, K, I, cfg["n_shared"], cfg["score_func"], cfg["renorm"], cfg["routed_scale"],
                    cfg["n_group"], cfg["topk_group"], 3, 256, 8, 1, _ot(rts[L]), ptr(bias, fp),
                    _ot(sh[0]), _ot(sh[1]), _ot(sh[2]), ptr(bT, fp), 9, recs, rb)
        rc, oi, ow, _ = orc.route(lgh[i], bias, E, K, cfg["score_func"], cfg["renorm"], cfg["routed_scale"],
                                  cfg["n_group"], cfg["topk_group"])
        assert rc == K
        assert np.array_equal(oi, idh[t, L]) and np.array_equal(bits(ow), bits(wh[t, L])), (t, L)
        xf = np.ascontiguousarray(xh[t, L].reshape(1, H))
        out = np.zeros((1, H), np.float32)
        rc = orc.lib.orc_moe_apply(C.byref(om), ptr(xf, fp), 1,
                                   np.ascontiguousarray(idh[t, L]).ctypes.data_as(C.POINTER(C.c_int)),
                                   ptr(np.ascontiguousarray(wh[t, L]), fp), 0, ptr(out, fp))
        assert rc == 0
        e_ = rel_err(yh[t, L].reshape(1, H), out)
        worst = max(worst, e_)
        assert e_ <= LAYER_RTOL, (t, L, e_)
    say(f"  {len(sample)} sampled layer outputs, worst rel err {worst:.2e}")
    for m in layers:
        m.close()
    cache.close()
    del host, X
