# SPDX-License-Identifier: Apache-2.0
"""The measured workloads at their own shapes, and the code paths the
benchmark shapes do not reach, against the oracle on an MI355X.

  DeepSeek-V3 512-token prefill chunk (Zipf(1.1) routing, and every token
  on eight hot experts): every token's ids and weights bit-exact against
  the oracle's router on the device's logits, every logit within 1e-5,
  and the outputs of >= 64 tokens (the longest segments' tokens, the
  singletons' and others) within 1e-3 of the oracle's moe_chunk order.
  Widths whose position count is not a multiple of 32 (the row-lane apply
  kernels, the separate SwiGLU pass and the scale-in-combine path) and
  batch-1 routing with more than 256 experts (the counter-ordered router
  launch): outputs within 1e-3, ids bit-exact.
  Three DeepSeek-V3 layers at full shape through an expert cache smaller
  than their working set: every output within 1e-3 of the oracle, the
  cache's decisions equal to its dry replay.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import ecache_script as es
from gpu_util import LAYER_RTOL, LOGIT_RTOL, gpu_layer, rel_err, run_forward
from oracle_lib import Oracle, OrcMoe, fp, ptr, u8p
from records import FMT_F32, FMT_Q4G, FMT_Q8G, Layer

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402
from warp_amd import synth  # noqa: E402
from test_gpu_fullsize import FullLayer, _ot, bits  # noqa: E402
from test_gpu_parity import check_routing  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


def pick_tokens(ids, n=64, seed=0):
    """Tokens whose outputs are compared: those of the three longest
    segments, those that own a singleton segment, and a spread of others,
    n in all (fewer when T is smaller)."""
    T = ids.shape[0]
    cnt = np.bincount(ids.reshape(-1), minlength=int(ids.max()) + 1)
    rng = np.random.default_rng(seed)
    chosen = []
    for e in np.argsort(-cnt, kind="stable")[:3]:
        toks = np.nonzero((ids == e).any(1))[0]
        chosen += rng.choice(toks, size=min(8, len(toks)), replace=False).tolist()
    single = np.nonzero(cnt == 1)[0]
    toks = sorted(set(np.nonzero(np.isin(ids, single).any(1))[0].tolist()))
    chosen += rng.choice(toks, size=min(24, len(toks)), replace=False).tolist() if toks else []
    chosen += [0, T - 1]
    rest = [t for t in range(T) if t not in set(chosen)]
    need = max(0, n - len(set(chosen)))
    chosen += rng.choice(rest, size=min(need, len(rest)), replace=False).tolist()
    return np.array(sorted(set(chosen)), np.int64), int(len(single))


def _prefill_case(orc, hot):
    T = 512
    L = FullLayer("dsv3", T)
    try:
        x = torch.from_numpy(synth.zipf_tokens(L.router, T, seed=7))
        if hot:
            b = L.bias.copy()
            gs = L.E // L.cfg["n_group"]
            b[[g * gs + o for g in (0, 2, 5, 7) for o in (1, gs - 2)]] += 5.0
            L.m.set_router(L.router, b)
            L.bias = b
        x = x.to(torch.bfloat16)
        st, y, ids, w, lg = L.forward(x)
        assert st == 0
        xf = np.ascontiguousarray(x.to(torch.float32).numpy())
        cnt = np.bincount(ids.reshape(-1), minlength=L.E)
        say(f"  T={T}: {int((cnt > 0).sum())} experts touched, {int((cnt >= 128).sum())} with >= 128 "
            f"tokens, longest segment {int(cnt.max())}")
        if hot:
            assert int((cnt >= 128).sum()) == 8
        # every token's routing, bit for bit, on the device's logits
        for t in range(T):
            rc, oi, ow, _ = orc.route(lg[t], L.bias, L.E, L.K, L.cfg["score_func"], L.cfg["renorm"],
                                      L.cfg["routed_scale"], L.cfg["n_group"], L.cfg["topk_group"])
            assert rc == L.K
            assert np.array_equal(oi, ids[t]), (t, oi, ids[t])
            assert np.array_equal(bits(ow), bits(w[t])), t
        # every token's logits
        om = L.oracle(orc, [])
        ref_lg = np.zeros((T, L.E), np.float32)
        orc.lib.orc_router_logits(C.byref(om), ptr(xf, fp), T, ptr(ref_lg, fp))
        e_lg = rel_err(lg, ref_lg)
        assert e_lg <= LOGIT_RTOL, e_lg
        # outputs of the chosen tokens (moe_chunk's order: ascending expert
        # id per token, zero weights skipped, the shared expert as a matmul)
        sel, n_single = pick_tokens(ids)
        om = L.oracle(orc, ids[sel].reshape(-1))
        out = np.zeros((len(sel), L.H), np.float32)
        xs = np.ascontiguousarray(xf[sel])
        rc = orc.lib.orc_moe_apply(C.byref(om), ptr(xs, fp), len(sel),
                                   np.ascontiguousarray(ids[sel]).ctypes.data_as(C.POINTER(C.c_int)),
                                   ptr(np.ascontiguousarray(w[sel]), fp), 1, ptr(out, fp))
        assert rc == 0
        e = rel_err(y[sel], out)
        per_tok = max(rel_err(y[t], out[i]) for i, t in enumerate(sel))
        say(f"  {len(sel)} tokens checked ({n_single} singleton segments): logits {e_lg:.2e}, "
            f"layer rel err {e:.3e}, worst token {per_tok:.3e}")
        assert len(sel) >= 64
        assert e <= LAYER_RTOL
    finally:
        L.close()


def test_dsv3_prefill_512_zipf(orc):
    say("test_dsv3_prefill_512_zipf")
    _prefill_case(orc, hot=False)


def test_dsv3_prefill_512_hot(orc):
    say("test_dsv3_prefill_512_hot")
    _prefill_case(orc, hot=True)


@pytest.mark.parametrize("H,I,T", [(2048, 1408, 1), (2048, 1408, 4), (1088, 512, 1), (1088, 512, 6),
                                   (1024, 448, 1), (1024, 448, 12)])
def test_row_lane_widths(orc, H, I, T):
    """Widths whose position count (H/8 or I/8) is not a multiple of 32, or
    whose row count (I for gate/up, H for down) is an odd number of 64-row
    blocks, run the row-lane apply kernels, the separate SwiGLU pass and the
    scales in the combine."""
    say("test_row_lane_widths", H, I, T)
    L = Layer(H, I, 16, 4, score_func=0, renorm=1, routed_scale=2.5, bias=True, n_shared=1,
              shared_fmt=FMT_Q8G, router_fmt=FMT_F32, seed=600 + I + T)
    X = L.inputs(T, seed=601)
    m = gpu_layer(L, max_tokens=T)
    st, y, ids, w, lg = run_forward(torch, m, L, X, False)
    m.close()
    assert st == 0
    ol = orc.moe(L, 1)
    assert rel_err(lg, ol.logits(X)) <= LOGIT_RTOL
    check_routing(orc, L, lg, ids, w)
    rc, ref = ol.apply(X, ids, w, chunk=int(T > 1))
    assert rc == 0
    e = rel_err(y, ref)
    say(f"  H={H} I={I} T={T}: layer rel err {e:.3e}")
    assert e <= LAYER_RTOL


@pytest.mark.parametrize("E,n_group,topk_group,score", [(384, 1, 1, 0), (512, 8, 4, 0), (320, 1, 1, 1)])
def test_batch1_routing_many_experts(orc, E, n_group, topk_group, score):
    """Batch 1 with more than 256 experts: the router launch's last block
    to count itself routes (the epoch exchange takes up to 256)."""
    say("test_batch1_routing_many_experts", E, n_group, topk_group, score)
    L = Layer(1024, 256, E, 8, score_func=score, renorm=1, routed_scale=2.5, bias=score == 0,
              n_group=n_group, topk_group=topk_group, n_shared=1, shared_fmt=FMT_Q4G,
              router_fmt=FMT_F32, seed=700 + E)
    ol = orc.moe(L, 1)
    m = gpu_layer(L)
    for t in range(3):
        X = L.inputs(1, seed=701 + t)
        st, y, ids, w, lg = run_forward(torch, m, L, X, False)
        assert st == 0
        assert rel_err(lg, ol.logits(X)) <= LOGIT_RTOL
        check_routing(orc, L, lg, ids, w)
        rc, ref = ol.apply(X, ids, w, chunk=0)
        assert rc == 0
        e = rel_err(y, ref)
        say(f"  E={E} token {t}: layer rel err {e:.3e}")
        assert e <= LAYER_RTOL
    m.close()


def test_dsv3_stack_through_cache(orc):
    """Three DeepSeek-V3 layers at full shape (16.5 MB records, 256 experts
    each) through an expert cache of 20 slots, below the 24 records one
    token needs: every layer output against the oracle, decisions against
    the dry replay of the same calls."""
    say("test_dsv3_stack_through_cache")
    cfg = synth.CONFIGS["dsv3"]
    H, E, K, I = cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]
    n_layers, T, n_slots, look = 3, 5, 20, 6
    dev = torch.device("cuda:0")
    rb = synth.record_bytes(H, I)
    books = synth.codebooks(0, H, I)
    host = torch.empty((n_layers * E, rb), dtype=torch.uint8, pin_memory=True)
    tmp = torch.empty(E * rb, dtype=torch.uint8, device=dev)
    trunks, ms = [], []
    for l in range(n_layers):
        synth.records(100 + l, l, H, I, books, 0, E, tmp.data_ptr())
        host[l * E:(l + 1) * E] = tmp.view(E, rb).cpu()
        router, bias, sh = synth.trunk(cfg, 200 + l)
        trunks.append((router, bias, sh))
        m = warp_amd.MoeLayer(hidden=H, n_experts=E, top_k=K, moe_inter=I, n_shared=cfg["n_shared"],
                              score_func=cfg["score_func"], renorm=cfg["renorm"],
                              routed_scale=cfg["routed_scale"], n_group=cfg["n_group"],
                              topk_group=cfg["topk_group"], layer=l, max_tokens=1)
        m.set_codebooks(books)
        m.set_router(router, bias)
        m.set_shared(*sh)
        assert m.bind_table([], [], codebook_id=0) == 0
        ms.append(m)
    del tmp
    torch.cuda.empty_cache()
    say(f"  {n_layers} layers of {E} records ({rb} B) in pinned host memory")
    cache = warp_amd.ExpertCache(rb, n_slots * rb, policy=0, depth=2)
    cache.set_source([host.data_ptr() + i * rb for i in range(n_layers * E)], n_layers, E)
    recs = (u8p * (n_layers * E))(*[C.cast(host.data_ptr() + i * rb, u8p) for i in range(n_layers * E)])
    _, bT = orc.books(books)
    oms = []
    for l in range(n_layers):
        router, bias, sh = trunks[l]
        oms.append(OrcMoe(H, E, K, I, cfg["n_shared"], cfg["score_func"], cfg["renorm"], cfg["routed_scale"],
                          cfg["n_group"], cfg["topk_group"], 3, 256, 8, 1, _ot(router), ptr(bias, fp),
                          _ot(sh[0]), _ot(sh[1]), _ot(sh[2]), ptr(bT, fp), 9,
                          C.cast(C.addressof(recs) + l * E * C.sizeof(u8p), C.POINTER(u8p)), rb))
    s = torch.cuda.current_stream().cuda_stream
    ops = []
    look_d = torch.empty((64,), dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(9)
    worst = 0.0
    for t in range(T):
        for l in range(n_layers):
            x = torch.randn((1, H), generator=g).to(torch.bfloat16)
            xd = x.to(dev)
            y = torch.full((1, H), float("nan"), device=dev)
            ids = torch.empty((1, K), dtype=torch.int32, device=dev)
            w = torch.empty((1, K), device=dev)
            nxt = ms[l + 1] if l + 1 < n_layers else None
            ms[l].forward_cached(cache, l, xd.data_ptr(), y.data_ptr(), nxt=nxt, lookahead=look,
                                 ids_ptr=ids.data_ptr(), w_ptr=w.data_ptr(), bf16=True, stream=s)
            assert ms[l].status(s) == 0, (t, l)
            idh = ids.cpu().numpy()[0].tolist()
            ops += [es.HINT, l, K] + idh
            for e in idh:
                ops += [es.HOLD, l, e]
            ops += [es.RELEASE]
            if nxt is not None:
                nxt.predict(xd.data_ptr(), look, look_d.data_ptr(), bf16=True, stream=s)
                gs = look_d.cpu().numpy()[:look].tolist()
                ops += [es.PREFETCH, l + 1, len(gs)] + gs
            xf = np.ascontiguousarray(x.to(torch.float32).numpy())
            out = np.zeros((1, H), np.float32)
            rc = orc.lib.orc_moe_apply(C.byref(oms[l]), ptr(xf, fp), 1,
                                       np.ascontiguousarray(ids.cpu().numpy()).ctypes.data_as(C.POINTER(C.c_int)),
                                       ptr(np.ascontiguousarray(w.cpu().numpy()), fp), 0, ptr(out, fp))
            assert rc == 0
            e_ = rel_err(y.cpu().numpy(), out)
            worst = max(worst, e_)
            assert e_ <= LAYER_RTOL, (t, l, e_)
    cache.sync()
    got = cache.stats()
    dry = warp_amd.ExpertCache(rb, n_slots * rb, policy=0, depth=2, dry=True)
    _, dst = es.run_product(dry, ops)
    assert [got[k] for k in ("hits", "misses", "evictions", "prefetched", "spec_issued", "reads")] == dst
    assert got["evictions"] > 0
    say(f"  hits {got['hits']} misses {got['misses']} evictions {got['evictions']} spec "
        f"{got['spec_issued']}, worst layer rel err {worst:.2e}")
    for m in ms:
        m.close()
    cache.close()
