# SPDX-License-Identifier: Apache-2.0
"""Layers loaded from a container directory, on an MI355X, through the C ABI.

The container is written by tests/container_writer.py in the reference's
format (two DeepSeek-V3-shaped MoE layers after one dense layer) and read
back by waste_hip_container_moe with the checksum on.

  against the oracle   built from what the container holds (its codebooks,
                       records and trunk tensors as the reader returns
                       them): ids and weights bit-exact on the device
                       logits, outputs within 1e-3, at T = 1, 8 and a
                       matrix-core prefill of 64 tokens
  against a direct     the same layer set up from the writer's arrays
  layer                (waste_hip_moe_set_*): bit-identical outputs
  group limit          off (the engine's moe_layer) and on (the config's
                       n_group / topk_group)
  through the cache    records left unbound, read into pinned memory with
                       read_bank and served by the HBM cache:
                       bit-identical to the layer's own slab
"""
import sys
import types

import numpy as np
import pytest

from container_writer import build, oracle_view, write
from gpu_util import LAYER_RTOL, LOGIT_RTOL, gpu_layer, rel_err, run_forward
from oracle_lib import Oracle
from records import FMT_F32, FMT_Q4G, Layer

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


@pytest.fixture(scope="module")
def ctr(tmp_path_factory):
    Ls = [Layer(1024, 256, 64, 8, score_func=0, renorm=1, routed_scale=2.5, bias=True, n_group=8,
                topk_group=4, n_shared=1, shared_fmt=FMT_Q4G, router_fmt=FMT_F32, seed=500 + r,
                cb_base=9 * r, layer=1 + r, subnormal_books=32) for r in range(2)]
    manifest, files = build(Ls, n_layers=3, first_dense=1)
    path = write(str(tmp_path_factory.mktemp("ctr")), manifest, files)
    return Ls, path


@pytest.mark.parametrize("T,prefill_min,group_limit", [(1, 0, False), (1, 0, True), (8, 0, False),
                                                       (64, 16, True)])
def test_container_layer(orc, ctr, T, prefill_min, group_limit):
    Ls, path = ctr
    say("test_container_layer", T, prefill_min, group_limit)
    c = warp_amd.Container(path, verify=True)
    for r, Lw in enumerate(Ls):
        layer = 1 + r
        ref = oracle_view(c, layer, group_limit)
        X = Lw.inputs(T, seed=900 + T + r)
        X = torch.from_numpy(X).to(torch.bfloat16).to(torch.float32).numpy()
        m = c.moe(layer, max_tokens=T, prefill_min_tokens=prefill_min, group_limit=group_limit)
        st, y, ids, w, lg = run_forward(torch, m, ref, X, bf16=True)
        assert st == 0
        ol = orc.moe(ref, 1)
        assert rel_err(lg, ol.logits(X)) <= LOGIT_RTOL
        for t in range(T):
            rc, oi, ow, _ = orc.route(lg[t], ref.bias, ref.E, ref.K, ref.score_func, ref.renorm,
                                      ref.routed_scale, ref.n_group, ref.topk_group)
            assert rc == ref.K
            assert np.array_equal(oi, ids[t]) and np.array_equal(bits(ow), bits(w[t])), (layer, t)
        rc, yref = ol.apply(X, ids, w, chunk=0 if T == 1 else 1)
        assert rc == 0
        e = rel_err(y, yref)
        say(f"  layer {layer} T={T}: rel err {e:.3e}")
        assert e <= LAYER_RTOL
        # the same layer from the writer's arrays, bit for bit
        Ld = types.SimpleNamespace(**vars(Lw))
        Ld.n_group, Ld.topk_group = ref.n_group, ref.topk_group
        md = gpu_layer(Ld, max_tokens=T, prefill_min=prefill_min)
        st2, y2, ids2, w2, lg2 = run_forward(torch, md, Ld, X, bf16=True)
        assert st2 == 0
        assert np.array_equal(bits(y), bits(y2)) and np.array_equal(ids, ids2)
        assert np.array_equal(bits(w), bits(w2)) and np.array_equal(bits(lg), bits(lg2))
        m.close()
        md.close()
    assert c.error()[0] == 0
    c.close()


def test_container_layer_through_cache(orc, ctr):
    """Unbound container layers fed by the HBM cache from read_bank's pinned
    copies equal the layers holding their own records, bit for bit."""
    Ls, path = ctr
    say("test_container_layer_through_cache")
    c = warp_amd.Container(path, verify=True)
    n, _, rb = c.bank(1)
    host = torch.empty((2 * n, rb), dtype=torch.uint8, pin_memory=True)
    for r in range(2):
        part = host[r * n:(r + 1) * n]
        assert c.read_bank(1 + r, (part.data_ptr(), part.numel())) == 0
    cache = warp_amd.ExpertCache(rb, 20 * rb, policy=0, depth=2)
    # cache keys are the engine's layer ids: 1 and 2; layer 0 has no bank
    ptrs = [0] * (n) + [host.data_ptr() + i * rb for i in range(2 * n)]
    cache.set_source(ptrs, 3, n)
    own = [c.moe(1 + r) for r in range(2)]
    fed = [c.moe(1 + r, records=False) for r in range(2)]
    for r, m in enumerate(fed):
        assert m.bind_table([], [], codebook_id=9 * r) == 0
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    for t in range(6):
        for r in range(2):
            x = Ls[r].inputs(1, seed=3000 + 10 * t + r)
            xd = torch.from_numpy(x).to(dev).to(torch.bfloat16)
            ya = torch.full((1, 1024), float("nan"), device=dev)
            yb = torch.full((1, 1024), float("nan"), device=dev)
            ia = torch.empty((1, 8), dtype=torch.int32, device=dev)
            ib = torch.empty((1, 8), dtype=torch.int32, device=dev)
            own[r].forward(xd.data_ptr(), 1, ya.data_ptr(), ia.data_ptr(), None, None, bf16=True, stream=s)
            nxt = fed[r + 1] if r == 0 else None
            fed[r].forward_cached(cache, 1 + r, xd.data_ptr(), yb.data_ptr(), nxt=nxt, lookahead=4 if nxt else 0,
                                  ids_ptr=ib.data_ptr(), bf16=True, stream=s)
            assert own[r].status(s) == 0 and fed[r].status(s) == 0
            assert np.array_equal(ia.cpu().numpy(), ib.cpu().numpy()), (t, r)
            assert np.array_equal(bits(ya.cpu().numpy()), bits(yb.cpu().numpy())), (t, r)
    cache.sync()
    st = cache.stats()
    say(f"  hits {st['hits']} misses {st['misses']}")
    assert st["misses"] > 0
    for m in own + fed:
        m.close()
    cache.close()
    c.close()


@pytest.mark.parametrize("T", [1, 4])
def test_reference_written_container_layers(orc, tmp_path, T):
    """The three MoE layers of the container the reference's own tool
    wrote (tests/golden/ref_container.npz, hidden 128, 8 experts, top-2,
    sigmoid with a bias, a Q4G router and shared expert) as device layers
    through the reader: ids and weights bit-exact on the device logits,
    outputs within 1e-3 of the oracle built from the reader's view."""
    from test_container import ref_container
    say("test_reference_written_container_layers", T)
    path, _ = ref_container(tmp_path)
    c = warp_amd.Container(path, verify=True)
    for layer in (1, 2, 3):
        ref = oracle_view(c, layer, False)
        X = np.random.default_rng(700 + layer + T).standard_normal((T, ref.H)).astype(np.float32)
        X = torch.from_numpy(X).to(torch.bfloat16).to(torch.float32).numpy()
        m = c.moe(layer, max_tokens=T)
        st, y, ids, w, lg = run_forward(torch, m, ref, X, bf16=True)
        assert st == 0
        ol = orc.moe(ref, 1)
        assert rel_err(lg, ol.logits(X)) <= LOGIT_RTOL
        for t in range(T):
            rc, oi, ow, _ = orc.route(lg[t], ref.bias, ref.E, ref.K, ref.score_func, ref.renorm,
                                      ref.routed_scale, ref.n_group, ref.topk_group)
            assert rc == ref.K
            assert np.array_equal(oi, ids[t]) and np.array_equal(bits(ow), bits(w[t])), (layer, t)
        rc, yref = ol.apply(X, ids, w, chunk=0 if T == 1 else 1)
        assert rc == 0
        e = rel_err(y, yref)
        say(f"  layer {layer} T={T}: rel err {e:.3e}")
        assert e <= LAYER_RTOL
        m.close()
    assert c.error()[0] == 0
    c.close()
