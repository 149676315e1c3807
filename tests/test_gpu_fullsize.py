# SPDX-License-Identifier: Apache-2.0
"""Full-size layers on the MI355X, checked against the oracle.

Layers are the benchmark shapes (OLMoE, Kimi-Linear, DeepSeek-V3), generated
on the device (waste_hip_synth_records: N(0,0.02) weights VQ3R-encoded
against seeded codebooks).  The oracle reads the routed experts' records
copied back to the host.

Bars: expert ids/weights bit-exact against the oracle's router on the
device's logits; router logits max rel error 1e-5; layer output max rel
error 1e-3 on the same routing; and the synthetic encoder's
stage indices are the nearest entries, checked by brute force.
"""
import ctypes as C
import sys

import numpy as np
import pytest

from gpu_util import LAYER_RTOL, LOGIT_RTOL, rel_err
from oracle_lib import Oracle, OrcMoe, OrcTensor, fp, ptr, u16p, u8p

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
import warp_amd  # noqa: E402
from warp_amd import synth  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return Oracle()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _ot(t):
    if t is None or t.rows == 0:
        return OrcTensor(0, 0, 0, 0, None, None, 0)
    return OrcTensor(t.fmt, t.rows, t.cols, t.group, t.q.ctypes.data_as(C.c_void_p),
                     ptr(t.qs, u16p) if t.qs is not None else None, t.rowbytes)


class FullLayer:
    def __init__(self, name, max_tokens, seed=0):
        cfg = self.cfg = synth.CONFIGS[name]
        self.H, self.E, self.K, self.I = cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]
        self.books = synth.codebooks(seed, self.H, self.I)
        self.rb = synth.record_bytes(self.H, self.I)
        self.slab = torch.empty(self.E * self.rb, dtype=torch.uint8, device="cuda:0")
        synth.records(seed, 0, self.H, self.I, self.books, 0, self.E, self.slab.data_ptr())
        self.router, self.bias, self.sh = synth.trunk(cfg, seed + 1)
        m = self.m = warp_amd.MoeLayer(hidden=self.H, n_experts=self.E, top_k=self.K, moe_inter=self.I,
                                       n_shared=cfg["n_shared"], score_func=cfg["score_func"],
                                       renorm=cfg["renorm"], routed_scale=cfg["routed_scale"],
                                       n_group=cfg["n_group"], topk_group=cfg["topk_group"],
                                       max_tokens=max_tokens)
        m.set_codebooks(self.books)
        m.set_router(self.router, self.bias)
        if self.sh:
            m.set_shared(*self.sh)
        for e in range(self.E):
            assert m.bind_expert(e, self.slab.data_ptr() + e * self.rb, self.rb) == 0

    def tokens(self, T, seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn((T, self.H), generator=g)
        if self.cfg["bf16"]:
            x = x.to(torch.bfloat16)
        return x

    def forward(self, x):
        T = x.shape[0]
        xd = x.to("cuda:0")
        y = torch.empty((T, self.H), dtype=torch.float32, device="cuda:0")
        ids = torch.empty((T, self.K), dtype=torch.int32, device="cuda:0")
        w = torch.empty((T, self.K), dtype=torch.float32, device="cuda:0")
        lg = torch.empty((T, self.E), dtype=torch.float32, device="cuda:0")
        s = torch.cuda.current_stream().cuda_stream
        self.m.forward(xd.data_ptr(), T, y.data_ptr(), ids.data_ptr(), w.data_ptr(), lg.data_ptr(),
                       bf16=self.cfg["bf16"], stream=s)
        st = self.m.status(s)
        return st, y.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), lg.cpu().numpy()

    def oracle(self, orc, experts):
        """OrcMoe over the given experts' records (others NULL)."""
        self.host = {}
        for e in sorted(set(int(v) for v in experts)):
            self.host[e] = self.slab[e * self.rb:(e + 1) * self.rb].cpu().numpy()
        ptrs = [ptr(self.host[e], u8p) if e in self.host else None for e in range(self.E)]
        self.recs = (u8p * self.E)(*ptrs)
        _, self.bT = orc.books(self.books)
        cfg = self.cfg
        return OrcMoe(self.H, self.E, self.K, self.I, cfg["n_shared"], cfg["score_func"], cfg["renorm"],
                      cfg["routed_scale"], cfg["n_group"], cfg["topk_group"], 3, 256, 8, 1,
                      _ot(self.router), ptr(self.bias, fp) if self.bias is not None else None,
                      _ot(self.sh[0] if self.sh else None), _ot(self.sh[1] if self.sh else None),
                      _ot(self.sh[2] if self.sh else None), ptr(self.bT, fp), 9, self.recs, self.rb)

    def close(self):
        self.m.close()
        del self.slab
        torch.cuda.empty_cache()


def check_layer(orc, L, x, chunk, ncheck=None):
    st, y, ids, w, lg = L.forward(x)
    assert st == 0
    T = x.shape[0]
    nt = T if ncheck is None else min(T, ncheck)
    om = L.oracle(orc, ids[:nt].reshape(-1))
    xf = np.ascontiguousarray(x.to(torch.float32).numpy())
    ref_lg = np.zeros((nt, L.E), np.float32)
    orc.lib.orc_router_logits(C.byref(om), ptr(xf, fp), nt, ptr(ref_lg, fp))
    assert rel_err(lg[:nt], ref_lg) <= LOGIT_RTOL
    for t in range(nt):
        rc, oi, ow, _ = orc.route(lg[t], L.bias, L.E, L.K, L.cfg["score_func"], L.cfg["renorm"],
                                  L.cfg["routed_scale"], L.cfg["n_group"], L.cfg["topk_group"])
        assert np.array_equal(oi, ids[t]), (t, oi, ids[t])
        assert np.array_equal(bits(ow), bits(w[t]))
    out = np.zeros((nt, L.H), np.float32)
    rc = orc.lib.orc_moe_apply(C.byref(om), ptr(xf, fp), nt,
                               np.ascontiguousarray(ids[:nt]).ctypes.data_as(C.POINTER(C.c_int)),
                               ptr(np.ascontiguousarray(w[:nt]), fp), int(chunk), ptr(out, fp))
    assert rc == 0
    e = rel_err(y[:nt], out)
    say(f"  T={T}: layer rel err {e:.3e}, distinct experts {len(np.unique(ids))}")
    assert e <= LAYER_RTOL
    return ids


@pytest.mark.parametrize("name,batches", [("olmoe", [1]), ("kimi", [1, 4, 16]), ("dsv3", [1, 8, 32])])
def test_fullsize_decode(orc, name, batches):
    say("test_fullsize_decode", name, batches)
    L = FullLayer(name, max(batches))
    try:
        for T in batches:
            x = L.tokens(T, seed=1000 + T)
            check_layer(orc, L, x, chunk=T > 1)
    finally:
        L.close()


def test_synth_encoder(orc):
    """The device encoder's output is a valid record whose stage indices are
    the nearest book entries (squared L2, first minimum) of the normalised
    row vectors, and whose row scales are f16(max|w|)."""
    say("test_synth_encoder")
    H, I = 512, 256
    books = synth.codebooks(3, H, I)
    rb = synth.record_bytes(H, I)
    dst = torch.empty(2 * rb, dtype=torch.uint8, device="cuda:0")
    raw = torch.empty((I, H), dtype=torch.float32, device="cuda:0")
    synth.records(5, 0, H, I, books, 0, 2, dst.data_ptr(), 0.02, raw.data_ptr())
    rec = dst[:rb].cpu().numpy()
    R = raw.cpu().numpy()
    assert np.allclose(np.abs(R).max(1), 1.0)
    m = warp_amd.MoeLayer(hidden=H, n_experts=2, top_k=1, moe_inter=I)
    m.set_codebooks(books)
    assert m.bind_expert(0, dst.data_ptr(), rb) == 0
    assert m.bind_expert(1, dst.data_ptr() + rb, rb) == 0
    m.close()
    bk, _ = orc.books(books)
    nv = H // 8
    r = np.random.default_rng(0)
    for _ in range(300):
        row, v = int(r.integers(I)), int(r.integers(nv))
        x = R[row, v * 8:(v + 1) * 8].astype(np.float32).copy()
        base = 48 + ((row // 64) * nv + v) * 192 + (row % 64) * 3
        for s in range(3):
            C_ = bk[s]
            d = np.zeros(256, np.float32)
            for j in range(8):
                t = (x[j] - C_[:, j]).astype(np.float32)
                d = (d + t * t).astype(np.float32)
            best = int(np.argmin(d))
            assert rec[base + s] == best, (row, v, s)
            x = (x - C_[best]).astype(np.float32)
