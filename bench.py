# SPDX-License-Identifier: Apache-2.0
"""MoE layer decode benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps 100] [--warmup 20] [--config dsv3] [--batch 1]

A step is one MoE layer forward over one batch of synthetic tokens:
router logits -> group-limited top-8 -> VQ3R gate/up -> SwiGLU -> VQ3R
down -> weighted combine + shared expert, everything resident in HBM.

The workload is the DeepSeek-V3-shaped layer (hidden 7168, 256 routed
experts of width 2048 in 3-bit residual VQ, sigmoid + bias, 8 groups / 4
kept, top-8, routed scale 2.5, one 4-bit shared expert, F32 router, bf16
activations), batch 1, seed 0.  Steps cycle over --layers layer objects
that share one expert slab but each hold their own router and shared
expert, and every step routes a fresh token, so no step finds its weights
in the 256 MB Infinity Cache from the step before — as in a real decode,
where 58 other layers run between two visits to the same one.

Printed: one JSON line with the metric (MoE layer us/token at batch 1),
HBM GB/s of algorithmic bytes, the dominant kernel's roofline from HIP
events on its stream, and the reference CPU path (C restatement,
AVX-512, all threads) timed on this host on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0        # dense fp16 / bf16
METRIC = "MoE layer µs/token + HBM GB/s (% of peak) at batch 1; prefill tokens/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_layers(torch, warp_amd, synth, cfg, n_layers, max_tokens, seed=0, slab=None, books=None,
                 own_slabs=False):
    """n_layers layer objects of one shape.  They share one expert slab
    (slab/books given, or generated here), or with own_slabs each holds its
    own records (seed + layer), for shapes whose slab would fit the 256 MB
    Infinity Cache and so not be read from HBM on every visit."""
    H, E, I = cfg["hidden"], cfg["n_experts"], cfg["moe_inter"]
    t0 = time.time()
    if books is None:
        books = synth.codebooks(seed, H, I)
    rb = synth.record_bytes(H, I)
    slabs = []
    if own_slabs:
        for li in range(n_layers):
            sl = torch.empty(E * rb, dtype=torch.uint8, device="cuda:0")
            synth.records(seed + li, 0, H, I, books, 0, E, sl.data_ptr())
            slabs.append(sl)
    else:
        if slab is None:
            slab = torch.empty(E * rb, dtype=torch.uint8, device="cuda:0")
            synth.records(seed, 0, H, I, books, 0, E, slab.data_ptr())
        slabs = [slab] * n_layers
    torch.cuda.synchronize()
    log(f"[bench] {len(set(map(id, slabs)))} x {E} expert records ({E * rb / 1e9:.2f} GB each) ready "
        f"in {time.time() - t0:.1f}s")
    router, bias, sh = synth.trunk(cfg, seed + 1)
    layers = []
    for li in range(n_layers):
        m = warp_amd.MoeLayer(hidden=H, n_experts=E, top_k=cfg["top_k"], moe_inter=I,
                              n_shared=cfg["n_shared"], score_func=cfg["score_func"],
                              renorm=cfg["renorm"], routed_scale=cfg["routed_scale"],
                              n_group=cfg["n_group"], topk_group=cfg["topk_group"],
                              max_tokens=max_tokens)
        m.set_codebooks(books)
        m.set_router(router, bias)
        if sh:
            m.set_shared(*sh)
        for e in range(E):
            rc = m.bind_expert(e, slabs[li].data_ptr() + e * rb, rb)
            if rc != 0:
                raise RuntimeError(f"bind_expert {e}: {rc}")
        layers.append(m)
    log(f"[bench] {n_layers} layer objects ready in {time.time() - t0:.1f}s")
    return layers, slabs[0] if not own_slabs else slabs, books, rb, (router, bias, sh)


def run_decode(torch, cfg, layers, B, steps, warmup, seed=0):
    """Decode steps at batch B: each step one forward of a fresh batch of
    tokens through the next layer object (the objects cycled).  Returns the
    timing record (event-timed over the steps, then a second pass with the
    per-stage profile on) and the tokens."""
    H, K, I = cfg["hidden"], cfg["top_k"], cfg["moe_inter"]
    gen = torch.Generator(device="cpu").manual_seed(seed)
    x_all = torch.randn(((warmup + steps + 8) * B, H), generator=gen, dtype=torch.float32)
    if cfg["bf16"]:
        x_all = x_all.to(torch.bfloat16)
    xd = x_all.to("cuda:0")
    esz = xd.element_size()
    y = torch.empty((B, H), dtype=torch.float32, device="cuda:0")
    ids = torch.empty((warmup + steps, B, K), dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def step(i, rec_ids=True):
        m = layers[i % len(layers)]
        m.forward(xd.data_ptr() + i * B * H * esz, B, y.data_ptr(),
                  ids[i].data_ptr() if rec_ids else None, None, None, bf16=cfg["bf16"], stream=sp)

    def status():
        for m in layers:
            st = m.status(sp)
            if st != 0:
                raise RuntimeError(f"device error {st}")

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    status()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(warmup, warmup + steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / steps
    status()

    # algorithmic bytes: distinct experts per step from the routed ids
    ids_h = ids[warmup:].cpu().numpy()
    distinct = [len(np.unique(ids_h[s].reshape(-1))) for s in range(steps)]
    bytes_per_step = float(np.mean([layers[0].bytes(B, u) for u in distinct]))
    gbps = bytes_per_step / (ms_per_step * 1e-3) / 1e9

    # live per-stage timing, a second pass over the same steps with profiling
    # on: at batch 1 each stage's kernel carries its own start/stop events in
    # its dispatch (kernel time only, no launch gaps); otherwise events on
    # the forward's stream around each stage
    for m in layers:
        m.profile(True)
    for i in range(warmup, warmup + steps):
        step(i, rec_ids=False)
    torch.cuda.synchronize()
    tot, nfw = {}, 0
    for m in layers:
        n, st = m.profile_read()
        nfw += n
        for k, v in st.items():
            tot[k] = tot.get(k, 0.0) + v
        m.profile(False)
    stage_ms = {k: v / nfw for k, v in tot.items()}
    dom = max(("routed_gate_up", "routed_down"), key=lambda k: stage_ms[k])
    u_mean = float(np.mean(distinct))
    # per-launch algorithmic bytes of the dominant kernel: the index streams
    # it reads (gate+up of every routed expert, or down)
    idx_gu = I * (H // 8) * 3
    idx_d = H * (I // 8) * 3
    dom_bytes = (2 * idx_gu if dom == "routed_gate_up" else idx_d) * u_mean
    rec = {"us_per_token": round(ms_per_step * 1e3 / B, 2), "ms_per_step": round(ms_per_step, 5),
           "hbm_gbps": round(gbps, 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
           "bytes_per_step": int(bytes_per_step), "distinct_experts_per_step": round(u_mean, 2),
           "wall_ms_per_step": round(wall * 1e3 / steps, 5),
           "stage_us": {k: round(v * 1e3, 2) for k, v in stage_ms.items()},
           "dominant": {"stage": dom, "kernel": "k_vq_gate_up" if dom == "routed_gate_up" else "k_vq_act_down",
                        "launch_us": round(stage_ms[dom] * 1e3, 2), "algorithmic_bytes": int(dom_bytes),
                        "achieved_gbps": round(dom_bytes / (max(stage_ms[dom], 1e-9) * 1e-3) / 1e9, 1)}}
    return rec, x_all


def host_cpu():
    """The host's CPU as lscpu states it (model, sockets x cores x threads),
    with the CPUs this process may run on and the physical cores among them
    (distinct (package, core) pairs in sysfs)."""
    import subprocess
    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass

    def num(k):
        try:
            return int(info[k])
        except (KeyError, ValueError):
            return None
    aff = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in aff:
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                cores.add((pkg, f.read().strip()))
        except OSError:
            cores = None
            break
    return {"model": info.get("Model name", "unknown"), "sockets": num("Socket(s)"),
            "cores_per_socket": num("Core(s) per socket"), "threads_per_core": num("Thread(s) per core"),
            "logical_cpus": num("CPU(s)"), "affinity_cpus": len(aff),
            "physical_cores_in_affinity": len(cores) if cores is not None else None}


def cpu_baseline(torch, cfg, slab, books, rb, trunk, xs, budget_s, nthreads):
    """The reference's CPU decode path (the oracle's AVX-512-order C
    restatement, threaded) on the same layer, timed on a bounded sample of
    the same tokens."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_lib import Oracle, OrcMoe, OrcTensor, fp, ptr, u16p, u8p
    import ctypes as C
    orc = Oracle()
    H, E, I, K = cfg["hidden"], cfg["n_experts"], cfg["moe_inter"], cfg["top_k"]
    host = slab.cpu().numpy()
    _, bT = orc.books(books)
    router, bias, sh = trunk

    def ot(t):
        if t is None or t.rows == 0:
            return OrcTensor(0, 0, 0, 0, None, None, 0)
        return OrcTensor(t.fmt, t.rows, t.cols, t.group, t.q.ctypes.data_as(C.c_void_p),
                         ptr(t.qs, u16p) if t.qs is not None else None, t.rowbytes)
    recs = (u8p * E)(*[ptr(host[e * rb:(e + 1) * rb], u8p) for e in range(E)])
    m = OrcMoe(H, E, K, I, cfg["n_shared"], cfg["score_func"], cfg["renorm"], cfg["routed_scale"],
               cfg["n_group"], cfg["topk_group"], 3, 256, 8, 1, ot(router),
               ptr(bias, fp) if bias is not None else None,
               ot(sh[0] if sh else None), ot(sh[1] if sh else None), ot(sh[2] if sh else None),
               ptr(bT, fp), 9, recs, rb)
    out = np.zeros(H, np.float32)
    idx = np.zeros(K, np.int32)
    w = np.zeros(K, np.float32)

    def timed(threads, budget):
        n, t_used = 0, 0.0
        first = True
        for i in range(1 << 20):               # the sample's tokens, cycled until the budget is spent
            x = np.ascontiguousarray(xs[i % len(xs)], np.float32)
            t0 = time.perf_counter()
            orc.lib.orc_moe_layer_mt(C.byref(m), ptr(x, fp), ptr(out, fp), idx.ctypes.data_as(C.POINTER(C.c_int)),
                                     ptr(w, fp), threads)
            dt = time.perf_counter() - t0
            if first:               # warm caches and the thread pool; not timed
                first = False
                continue
            n += 1
            t_used += dt
            if t_used >= budget and n >= 3:
                break
        return n, t_used
    n, t_used = timed(nthreads, budget_s)
    n1, t1 = timed(1, budget_s / 4)            # one thread, a quarter of the budget
    isa = {2: "AVX-512", 0: "portable C"}[orc.lib.orc_cpu_isa()]
    return n, t_used, isa, n1, t1


def bench_vq4p(torch, warp_amd, reps=64):
    """VQ4P rows through the int8 LUT (the vq_rows_p6 slot's kernel on device
    pointers) on the C3 shapes: gate/up (2048 rows x 896 positions) and down
    (7168 x 256).  Random codes (any byte triple is four 6-bit codes), a
    quantised random table; each launch reads its own matrix of `reps`, so
    the 256 MB Infinity Cache holds none of them from the launch before.
    Algorithmic bytes: the codes, 3 per (row, position), plus the f16 row
    scales and the int8 table."""
    L = warp_amd.lib()
    dev = "cuda:0"
    s = torch.cuda.current_stream()
    out = {}
    g = torch.Generator(device=dev).manual_seed(5)
    for name, M, nv in (("gate_up", 2048, 896), ("down", 7168, 256)):
        idx = torch.randint(0, 256, (reps, M * nv * 3), dtype=torch.uint8, device=dev, generator=g)
        sc = (torch.rand((M,), device=dev, generator=g) * 0.02 + 0.005).half()
        lut = torch.randn((nv * 256,), device=dev, generator=g)
        q = torch.empty((nv * 256,), dtype=torch.int8, device=dev)
        qs = torch.empty(((nv + 31) // 32,), dtype=torch.float32, device=dev)
        warp_amd.check(L.waste_hip_vq_quant_lut(lut.data_ptr(), nv, 4, 64, q.data_ptr(), qs.data_ptr(), s.cuda_stream),
                       "vq_quant_lut")
        y = torch.empty((M,), dtype=torch.float32, device=dev)

        def one(r):
            warp_amd.check(L.waste_hip_vq_rows_p6(idx[r].data_ptr(), sc.data_ptr(), q.data_ptr(), qs.data_ptr(), 0, M,
                                                  nv, 1, y.data_ptr(), s.cuda_stream), "vq_rows_p6")
        for r in range(reps):
            one(r)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for r in range(reps):
            one(r)
        e1.record(s)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = M * nv * 3 + M * 2 + nv * 256 + ((nv + 31) // 32) * 4
        out[name] = {"rows": M, "positions": nv, "us": round(us, 2), "bytes": nbytes,
                     "gbps": round(nbytes / (us * 1e-6) / 1e9, 1), "hbm_frac": round(nbytes / (us * 1e-6) / 8e12, 4)}
        del idx
    return out


def bench_prefill(torch, warp_amd, synth, cfg, slab, books, rb, trunk, T, reps, hot=False):
    """One T-token chunk of the layer (moe_chunk on the matrix cores).  Tokens
    are planted so per-expert counts follow Zipf(1.1) (synth.zipf_tokens), or
    with hot=True a bias sends every token to the same eight experts (two in
    each of four groups), so every routed group has T >= 128 tokens."""
    H, E, K, I = cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]
    router, bias, sh = trunk
    m = warp_amd.MoeLayer(hidden=H, n_experts=E, top_k=K, moe_inter=I, n_shared=cfg["n_shared"],
                          score_func=cfg["score_func"], renorm=cfg["renorm"],
                          routed_scale=cfg["routed_scale"], n_group=cfg["n_group"],
                          topk_group=cfg["topk_group"], max_tokens=T)
    m.set_codebooks(books)
    b = None if bias is None else bias.copy()
    if hot:
        gs = E // cfg["n_group"]
        b[[g * gs + o for g in (0, 2, 5, 7) for o in (1, gs - 2)]] += 5.0
    m.set_router(router, b)
    if sh:
        m.set_shared(*sh)
    for e in range(E):
        assert m.bind_expert(e, slab.data_ptr() + e * rb, rb) == 0
    X = synth.zipf_tokens(router, T, seed=7)
    xd = torch.from_numpy(X).to("cuda:0")
    if cfg["bf16"]:
        xd = xd.to(torch.bfloat16)
    y = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
    ids = torch.empty((T, K), dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    fwd = lambda: m.forward(xd.data_ptr(), T, y.data_ptr(), ids.data_ptr(), None, None, bf16=cfg["bf16"],
                            stream=sp)
    for _ in range(2):
        fwd()
    torch.cuda.synchronize()
    if m.status(sp) != 0:
        raise RuntimeError("prefill device error")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(reps):
        fwd()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / reps
    m.profile(True)
    for _ in range(reps):
        fwd()
    torch.cuda.synchronize()
    n, st = m.profile_read()
    m.profile(False)
    st = {k: v / n for k, v in st.items()}
    if m.status(sp) != 0:
        raise RuntimeError("prefill device error")
    ih = ids.cpu().numpy()
    cnt = np.bincount(ih.reshape(-1), minlength=E)
    U = int((cnt > 0).sum())
    P = T * K
    SI = I * max(cfg["n_shared"], 1)
    f_gu, f_d = 2.0 * P * 2 * I * H, 2.0 * P * H * I
    f_sh = 2.0 * T * 3 * SI * H if sh else 0.0
    f_all = f_gu + f_d + f_sh + 2.0 * T * E * H
    routed_ms = st["routed_gate_up"] + st["routed_down"]
    nbytes = m.bytes(T, U)
    m.close()
    return {
        "tokens": T, "routing": "8 hot experts (every routed group = all tokens)" if hot
        else "Zipf(1.1) planted logits, seed 7",
        "ms_per_chunk": round(ms, 3), "tokens_per_s": round(T / (ms * 1e-3), 1),
        "experts_touched": U, "experts_ge128": int((cnt >= 128).sum()),
        "pairs_in_ge128": round(float(cnt[cnt >= 128].sum()) / P, 3),
        "flops": f_all, "hbm_bytes": int(nbytes),
        "floor_ms": round(max(nbytes / (HBM_PEAK_GBPS * 1e9), f_all / (MFMA_PEAK_TFLOPS * 1e12)) * 1e3, 3),
        "routed_grouped_gemm": {"ms": round(routed_ms, 3),
                                "tflops": round((f_gu + f_d) / (routed_ms * 1e-3) / 1e12, 1),
                                "mfma_frac": round((f_gu + f_d) / (routed_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)},
        "stage_ms": {k: round(v, 3) for k, v in st.items()},
    }


def sticky_gumbel(rng, T, E, keep):
    """[T][E] Gumbel noise whose entries each carry over from the row before
    with probability keep (else a fresh draw): every row is Gumbel, and
    consecutive rows share about `keep` of their values."""
    g = np.empty((T, E))
    g[0] = rng.gumbel(size=E)
    for t in range(1, T):
        g[t] = np.where(rng.random(E) < keep, g[t - 1], rng.gumbel(size=E))
    return g


def stack_inputs(torch, routers, T, zipf_s, reuse_keep, look_keep, scale, seed, device="cuda:0"):
    """Tokens whose routing follows the stated workload, bf16 [T][L][H] on
    the device, and each layer's popularity ranks.

    Layer L's router logits for token t are planted as
    scale * (log p_L + g[t]) (less their expected mean): p_L ~ rank^-zipf_s over a seeded permutation of
    the experts, g sticky Gumbel noise (sticky_gumbel, reuse_keep).  With
    Gumbel noise the router's top-k is a draw without replacement from p_L
    (the Gumbel-max form), and the carried-over noise is what makes
    consecutive tokens reuse experts.  The next layer's router applied to
    the same token sees its own planted logits with only look_keep of the
    noise values in common, so the lookahead guesses as well as that
    overlap allows.  The token is the minimum-norm solution of both
    routers' equations (x = M^T (M M^T)^-1 [l_L; l_L+1~], M the two routers
    stacked) plus N(0,1) noise orthogonal to their rows, so every coordinate
    still looks like N(0,1) noise."""
    rng = np.random.default_rng(seed)
    n_layers = len(routers)
    E, H = routers[0].shape
    ranks = []
    for L in range(n_layers):
        rank = np.empty(E, np.int64)
        rank[rng.permutation(E)] = np.arange(E)
        ranks.append(rank)
    # log-popularity and the noise, both centred: a constant added to every
    # logit of a token changes no selection, and centred logits keep the
    # planted part of the token small
    lp = [-zipf_s * np.log(r + 1.0) for r in ranks]
    lp = [v - v.mean() - np.euler_gamma for v in lp]
    g = [sticky_gumbel(rng, T, E, reuse_keep) for _ in range(n_layers)]
    X = torch.empty((T, n_layers, H), dtype=torch.bfloat16, device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    for L in range(n_layers):
        own = scale * (lp[L] + g[L])                                     # [T][E]
        rows = [torch.from_numpy(routers[L]).to(device, torch.float64)]
        tg = [own]
        if L + 1 < n_layers:
            mix = np.where(rng.random((T, E)) < look_keep, g[L + 1], rng.gumbel(size=(T, E)))
            tg.append(scale * (lp[L + 1] + mix))
            rows.append(torch.from_numpy(routers[L + 1]).to(device, torch.float64))
        M = torch.cat(rows)                                              # [nE][H]
        Gm = M @ M.T
        tgt = torch.from_numpy(np.concatenate(tg, 1)).to(device, torch.float64)   # [T][nE]
        x = torch.linalg.solve(Gm, tgt.T).T @ M
        z = torch.randn((T, H), generator=gen, device=device, dtype=torch.float64)
        z -= torch.linalg.solve(Gm, (z @ M.T).T).T @ M
        X[:, L] = (x + z).to(torch.bfloat16)
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize()
    return X, ranks


def zipf_mle(counts_by_rank):
    """Maximum-likelihood Zipf exponent of counts indexed by rank (rank 1
    first), over every rank."""
    n = np.asarray(counts_by_rank, np.float64)
    r = np.arange(1, n.size + 1, dtype=np.float64)
    ss = np.arange(0.3, 2.5, 0.001)
    ll = [-s * float((n * np.log(r)).sum()) - n.sum() * np.log(float((r ** -s).sum())) for s in ss]
    return float(ss[int(np.argmax(ll))])


def stack_setup(torch, warp_amd, synth, cfg, books, tokens, n_layers=58, budget_gb=64.0, depth=2, seed=0,
                zipf_s=1.1, reuse_keep=0.63, look_keep=0.88, scale=0.5):
    """The stack bench_stack runs (see there): the host bank in pinned
    memory, n_layers layer objects with their own routers and the shared
    expert, the HBM expert cache over the bank, and the tokens.  Returns
    (layers, routers, cache, host, X [T][L][H] bf16, ranks, rec_bytes)."""
    H, E, I, K = cfg["hidden"], cfg["n_experts"], cfg["moe_inter"], cfg["top_k"]
    rb = synth.record_bytes(H, I)
    dev = torch.empty(E * rb, dtype=torch.uint8, device="cuda:0")
    synth.records(seed, 0, H, I, books, 0, E, dev.data_ptr())
    host = torch.empty(E * rb, dtype=torch.uint8, pin_memory=True)
    host.copy_(dev)
    del dev
    torch.cuda.synchronize()
    _, _, sh = synth.trunk(cfg, seed + 1)
    rng = np.random.default_rng(seed + 7)
    layers, routers = [], []
    for L in range(n_layers):
        W = (rng.standard_normal((E, H), np.float32) * 0.02).astype(np.float32)
        routers.append(W)
        b = np.zeros(E, np.float32)
        m = warp_amd.MoeLayer(hidden=H, n_experts=E, top_k=K, moe_inter=I,
                              n_shared=cfg["n_shared"], score_func=cfg["score_func"],
                              renorm=cfg["renorm"], routed_scale=cfg["routed_scale"],
                              n_group=cfg["n_group"], topk_group=cfg["topk_group"], layer=0,
                              max_tokens=1)
        m.set_codebooks(books)
        m.set_router(synth.Tensor.make(cfg["router_fmt"], W), b)
        if sh:
            m.set_shared(*sh)
        warp_amd.check(m.bind_table([], [], codebook_id=0), "bind_table")
        layers.append(m)
    cache = warp_amd.ExpertCache(rb, int(budget_gb * 1e9), policy=0, depth=depth)
    cache.set_source([host.data_ptr() + e * rb for _ in range(n_layers) for e in range(E)], n_layers, E)
    X, ranks = stack_inputs(torch, routers, tokens, zipf_s, reuse_keep, look_keep, scale, seed + 11)
    return layers, routers, cache, host, X, ranks, rb


def group_top(sc, n, n_group, topk_group):
    """The n best of scores sc [E] within the topk_group groups of the
    largest top-2 sums (the routing's group limit), best first."""
    g = sc.reshape(n_group, -1)
    keep = np.argsort(-np.sort(g, 1)[:, -2:].sum(1), kind="stable")[:topk_group]
    m = np.full(sc.shape, -np.inf)
    for k in keep:
        m[k * g.shape[1]:(k + 1) * g.shape[1]] = g[k]
    return np.argsort(-m, kind="stable")[:n]


def bench_stack(torch, warp_amd, synth, cfg, books, tokens, n_layers=58, budget_gb=64.0,
                lookahead=6, depth=2, seed=0, zipf_s=1.1, reuse_keep=0.63, look_keep=0.88, scale=0.5,
                grouped=False):
    """58 DeepSeek-V3-shaped MoE layers decoding `tokens` tokens at batch 1
    through the HBM expert cache (64 GB of slots), the expert records in
    pinned host memory, misses filled by hipMemcpyAsync on the cache's
    stream, the lookahead's guesses (the next layer's router on this
    layer's input, 6 ids) read after each layer's experts.  grouped: the
    guesses within the next layer's own group limit (8 groups, 4 kept)
    rather than the engine's rule (the top 6 over all experts).

    Routing (stack_inputs): each layer's experts drawn without replacement
    from Zipf(zipf_s) popularity over a seeded permutation, consecutive
    tokens sharing reuse_keep of the draw's noise (0.63: 0.6 of a token's
    experts reused by the next), the next layer's router on this layer's
    input sharing look_keep of it (0.88: about 81% of the top-6 guesses
    land and 92% of the first, the precision the engine measured on a real
    model, docs/LEARNED.md:1866-1868).  The e_score_correction_bias is
    present and zero.

    The host bank: one set of 256 records (4.2 GB pinned); layer L's expert
    e is a byte copy of record e, so every layer object carries layer id 0
    (the records' header) while the cache keys are (L, e): each miss still
    moves its own 16.5 MB over PCIe into its own slot."""
    H, E, I, K = cfg["hidden"], cfg["n_experts"], cfg["moe_inter"], cfg["top_k"]
    t0 = time.time()
    layers, routers, cache, host, X, ranks, rb = stack_setup(torch, warp_amd, synth, cfg, books, tokens, n_layers,
                                                             budget_gb, depth, seed, zipf_s, reuse_keep, look_keep,
                                                             scale)
    for m in layers:
        m.set_lookahead_groups(grouped)
    y = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    ids = torch.empty((tokens, n_layers, K), dtype=torch.int32, device="cuda:0")
    torch.cuda.synchronize()
    log(f"[bench] stack: {n_layers} layers, {cache.n_slots} slots of {rb} B, bank in pinned host "
        f"memory, set up in {time.time() - t0:.1f}s")
    s = torch.cuda.current_stream().cuda_stream
    esz = X.element_size()
    tok_s, marks = [], []
    t_start = time.perf_counter()
    for t in range(tokens):
        for L in range(n_layers):
            nxt = layers[L + 1] if L + 1 < n_layers else None
            layers[L].forward_cached(cache, L, X.data_ptr() + (t * n_layers + L) * H * esz, y.data_ptr(),
                                     nxt=nxt, lookahead=lookahead if nxt else 0,
                                     ids_ptr=ids[t, L].data_ptr(), bf16=True, stream=s)
        marks.append(time.perf_counter())
        if t % 50 == 49:
            st = cache.stats()
            log(f"[bench] stack token {t + 1}: hit rate {st['hits'] / max(1, st['hits'] + st['misses']):.3f}")
    torch.cuda.synchronize()
    cache.sync()
    wall = time.perf_counter() - t_start
    for m in layers:
        st = m.status(s)
        if st != 0:
            raise RuntimeError(f"stack: device error {st}")
    st = cache.stats()
    hit = st["hits"] / max(1, st["hits"] + st["misses"])
    half = tokens // 2
    steady = (tokens - half) / (marks[-1] - marks[half - 1]) if half else None
    # the routing the layers actually made
    ih = ids.cpu().numpy()
    reuse = float(np.mean([len(set(ih[t, L]) & set(ih[t - 1, L])) / K
                           for t in range(1, tokens) for L in range(n_layers)]))
    cnt = np.zeros((n_layers, E))
    by_rank, fresh_by_rank = np.zeros(E), np.zeros(E)
    for L in range(n_layers):
        np.add.at(cnt[L], ih[:, L].reshape(-1), 1)
        np.add.at(by_rank, ranks[L][ih[:, L].reshape(-1)], 1)
        for t in range(tokens):
            new = [e for e in ih[t, L] if t == 0 or e not in ih[t - 1, L]]
            np.add.at(fresh_by_rank, ranks[L][np.array(new, np.int64)], 1)
    # the lookahead's guesses: the next layer's router on this layer's
    # input, its top 6 by score (the bias is zero; grouped: within the
    # group limit), against what the next layer then selected
    hits6 = hits1 = n_guess = 0
    for L in range(n_layers - 1):
        Wn = torch.from_numpy(routers[L + 1]).to("cuda:0")
        sc = torch.sigmoid(X[:, L].float() @ Wn.T).cpu().numpy()
        for t in range(tokens):
            g = (group_top(sc[t], lookahead, cfg["n_group"], cfg["topk_group"]) if grouped
                 else np.argsort(-sc[t], kind="stable")[:lookahead])
            nxt_sel = set(ih[t, L + 1].tolist())
            hits6 += len(nxt_sel & set(g.tolist()))
            hits1 += int(g[0] in nxt_sel)
            n_guess += 1
    out = {
        "workload": f"{n_layers}-layer dsv3 MoE stack, batch-1 decode of {tokens} tokens through the "
                    f"HBM expert cache", "layers": n_layers, "tokens": tokens,
        "budget_gb": budget_gb, "slots": cache.n_slots, "records": n_layers * E, "rec_bytes": rb,
        "policy": "lfru", "readahead_depth": depth, "lookahead": lookahead,
        "lookahead_rule": "within the group limit" if grouped else "top n over all experts (predict_next_moe)",
        "hit_rate": round(hit, 4), "hits": st["hits"], "misses": st["misses"],
        "evictions": st["evictions"], "hint_reads": st["prefetched"],
        "lookahead_reads": st["spec_issued"],
        # what became of them: demanded while resident, evicted unread, or
        # still resident and unread when the run ended
        "lookahead_reads_used": st["spec_used"], "lookahead_reads_wasted": st["spec_wasted"],
        "lookahead_reads_unresolved": st["spec_issued"] - st["spec_used"] - st["spec_wasted"],
        "gb_read": round(st["bytes_read"] / 1e9, 2), "gb_read_per_token": round(st["bytes_read"] / 1e9 / tokens, 3),
        "tok_s": round(tokens / wall, 3), "ms_per_token": round(wall * 1e3 / tokens, 2),
        "tok_s_second_half": round(steady, 3) if steady else None,
        "host_to_device_gbps": round(st["bytes_read"] / wall / 1e9, 2),
        "routing": {"distinct_experts_per_layer": round(float((cnt > 0).sum(1).mean()), 1),
                    "token_to_token_reuse": round(reuse, 3),
                    "fresh_selections_per_layer": round(float(fresh_by_rank.sum()) / n_layers, 1),
                    "zipf_mle_all_ranks": round(zipf_mle(by_rank), 3),
                    "zipf_mle_fresh_all_ranks": round(zipf_mle(fresh_by_rank), 3),
                    "lookahead_precision_top6": round(hits6 / max(1, n_guess * lookahead), 3),
                    "lookahead_precision_rank1": round(hits1 / max(1, n_guess), 3),
                    "generator": {"popularity": f"Zipf({zipf_s}) over a seeded permutation per layer, "
                                                f"drawn without replacement (Gumbel top-k)",
                                  "reuse_keep": reuse_keep, "look_keep": look_keep, "logit_scale": scale}},
    }
    for m in layers:
        m.close()
    cache.close()
    del host, X
    return out


def bench_formats(torch, warp_amd, synth, cfg, n_layers, steps, warmup, batches=(1, 8)):
    """The other expert formats through the device layer at the C3 shape:
    VQ4P (index_bits 6: four stages of 64 entries, int8 tables, rows as
    vq_rows_p6) and VQ2R (two stages of 256 entries, fp32 tables, rows in
    vq_rows' order).  Both paths reproduce the engine's arithmetic exactly
    (the VQ3R tile kernels do not serve them).  One slab of 256 records with
    random codes (any byte pair or triple decodes to valid codes), valid
    headers and f16 row scales in [0.01, 0.05), shared by n_layers layer
    objects as the VQ3R step shares its slab; random books; the same router
    and shared expert."""
    import struct
    H, E, I, K = cfg["hidden"], cfg["n_experts"], cfg["moe_inter"], cfg["top_k"]
    nv_h, nv_i = H // 8, I // 8
    router, bias, sh = synth.trunk(cfg, 1)
    out = {}
    g = torch.Generator(device="cuda:0").manual_seed(11)
    for name, ib, st, en, bpp, fmt in (("vq4p", 6, 4, 64, 3, 8), ("vq2r", 8, 2, 256, 2, 5)):
        idx_gu, idx_d = I * nv_h * bpp, H * nv_i * bpp
        off_up, off_down, off_sc = 48 + idx_gu, 48 + 2 * idx_gu, 48 + 2 * idx_gu + idx_d
        rb = (off_sc + 2 * (2 * I + H) + 4095) // 4096 * 4096
        slab = torch.randint(0, 256, (E, rb), dtype=torch.uint8, device="cuda:0", generator=g)
        hdr = np.zeros((E, 48), np.uint8)
        for e in range(E):
            hdr[e] = np.frombuffer(struct.pack("<IHHBBHHHIIIIIIII", 0x50584557, 0, e, fmt, 0, 0, 0, 0, rb // 4096,
                                               48, off_up, off_down, off_sc, 0, 0, 0), np.uint8)
        slab[:, :48] = torch.from_numpy(hdr).to("cuda:0")
        sc = (torch.rand((E, 2 * I + H), device="cuda:0", generator=g) * 0.04 + 0.01).half()
        slab[:, off_sc:off_sc + 2 * (2 * I + H)] = sc.view(torch.uint8)
        rng = np.random.default_rng(12)
        books = synth.f16_bits((rng.standard_normal((3 * st, en, 8)) * 0.3).astype(np.float32))
        layers = []
        for _ in range(n_layers):
            m = warp_amd.MoeLayer(hidden=H, n_experts=E, top_k=K, moe_inter=I, n_shared=cfg["n_shared"],
                                  score_func=cfg["score_func"], renorm=cfg["renorm"],
                                  routed_scale=cfg["routed_scale"], n_group=cfg["n_group"],
                                  topk_group=cfg["topk_group"], max_tokens=max(batches), index_bits=ib,
                                  stages=st if ib == 8 else 0)
            m.set_codebooks(books)
            m.set_router(router, bias)
            if sh:
                m.set_shared(*sh)
            for e in range(E):
                rc = m.bind_expert(e, slab[e].data_ptr(), rb)
                if rc != 0:
                    raise RuntimeError(f"{name} bind_expert {e}: {rc}")
            layers.append(m)
        torch.cuda.synchronize()
        for bb in batches:
            r, _ = run_decode(torch, cfg, layers, bb, steps, warmup, seed=100 + bb)
            out[f"{name}_b{bb}"] = {k: r[k] for k in ("us_per_token", "ms_per_step", "hbm_gbps", "hbm_frac",
                                                     "bytes_per_step", "distinct_experts_per_step", "stage_us")}
            log(f"[bench] {name} B={bb}: {r['us_per_token']} us/token, {r['hbm_frac']:.3f} of HBM peak")
        for m in layers:
            m.close()
        del slab
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def measured_traffic(dom, config, batch):
    """HBM bytes per launch of the dominant kernel, as measured by the two
    rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE, each scaled by a copy of
    known size) whose summary is kept in profiles/; None without one."""
    kernel = "k_vq_gate_up" if dom == "routed_gate_up" else "k_vq_act_down"
    path = os.path.join(ROOT, "profiles", f"{kernel}-{config}-decode-b{batch}-hbm-traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="dsv3")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="tokens of the prefill chunk measured beside decode (0: skip)")
    ap.add_argument("--stack-tokens", type=int, default=200,
                    help="tokens the 58-layer stack decodes through the HBM expert cache (0: skip)")
    ap.add_argument("--stack-budget-gb", type=float, default=64.0)
    ap.add_argument("--no-stack-grouped", dest="stack_grouped", action="store_false",
                    help="skip the second stack run, whose lookahead guesses lie within the group limit")
    ap.add_argument("--no-extra-configs", dest="extra_configs", action="store_false",
                    help="skip the other decode configurations (olmoe B=1, kimi B=1/4/16, dsv3 B=8/32) "
                         "and the other record formats (VQ4P rows, VQ4P and VQ2R layers)")
    ap.add_argument("--no-decode-configs", dest="decode_configs", action="store_false",
                    help="skip the other decode configurations (C3 batch 8/32, C1, C2); the formats still run")
    ap.add_argument("--copy-calibrate", type=int, default=0, metavar="MB",
                    help="first copy MB megabytes device to device (a plain copy kernel of known "
                         "size, the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build's MoE path runs on a single MI355X and "
              f"--gpus {a.gpus} is not supported (expert-parallel sharding over several GPUs is not built).",
              file=sys.stderr)
        return 2

    import torch
    import warp_amd
    from warp_amd import synth
    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    cfg = synth.CONFIGS[a.config]
    H, E, K, I = cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]
    B = a.batch
    # a slab per layer object for the small shapes (as in the other
    # configurations below): one shared slab of theirs fits the Infinity Cache
    own = a.config != "dsv3"
    layers, slab, books, rb, trunk = build_layers(torch, warp_amd, synth, cfg, a.layers, B, own_slabs=own)
    slabs_own, slab = (slab, slab[0]) if own else (None, slab)
    if a.copy_calibrate:
        n = a.copy_calibrate << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {a.copy_calibrate} MiB device to device 3 times (counter scale)")
        del src, dst

    dec, x_all = run_decode(torch, cfg, layers, B, a.steps, a.warmup)
    ms_per_step = dec["ms_per_step"]
    us_per_token = dec["us_per_token"]
    dom = dec["dominant"]
    achieved = dom["achieved_gbps"]
    traffic = measured_traffic(dom["stage"], a.config, B)

    # the other decode configurations, each on its own layer objects: the
    # small shapes with a slab per object so the cycled records do not fit
    # the Infinity Cache
    per_config = None
    if a.extra_configs and a.decode_configs and B == 1 and a.config == "dsv3":
        per_config = []
        big = build_layers(torch, warp_amd, synth, cfg, a.layers, 32, slab=slab, books=books)[0]
        for bb in (8, 32):
            r, _ = run_decode(torch, cfg, big, bb, a.steps, a.warmup, seed=bb)
            per_config.append(dict(config="C3", workload=f"dsv3 MoE layer decode, batch {bb}", batch=bb, **r))
            log(f"[bench] C3 B={bb}: {r['us_per_token']} us/token, {r['hbm_frac']:.3f} of HBM peak")
        for m in big:
            m.close()
        del big
        for name, tag, batches in (("olmoe", "C1", (1,)), ("kimi", "C2", (1, 4, 16))):
            c2 = synth.CONFIGS[name]
            ls, slabs, _, _, _ = build_layers(torch, warp_amd, synth, c2, a.layers, max(batches),
                                              own_slabs=True)
            for bb in batches:
                r, _ = run_decode(torch, c2, ls, bb, a.steps, a.warmup, seed=bb)
                per_config.append(dict(config=tag, workload=f"{name} MoE layer decode, batch {bb}", batch=bb, **r))
                log(f"[bench] {tag} B={bb}: {r['us_per_token']} us/token, {r['hbm_frac']:.3f} of HBM peak")
            for m in ls:
                m.close()
            del ls, slabs
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    prefill = None
    if a.prefill_tokens and B == 1:
        prefill = bench_prefill(torch, warp_amd, synth, cfg, slab, books, rb, trunk, a.prefill_tokens, 5)
        prefill["ge128_groups"] = bench_prefill(torch, warp_amd, synth, cfg, slab, books, rb, trunk,
                                                a.prefill_tokens, 5, hot=True)["routed_grouped_gemm"]
        log(f"[bench] prefill {prefill['tokens_per_s']} tok/s")

    vq4p = formats = None
    if a.extra_configs and B == 1:
        vq4p = bench_vq4p(torch, warp_amd)
        formats = bench_formats(torch, warp_amd, synth, cfg, a.layers, a.steps, a.warmup) if a.config == "dsv3" else None
        log(f"[bench] vq4p rows: {vq4p}")

    stack = None
    if a.stack_tokens and B == 1 and a.config == "dsv3":
        stack = bench_stack(torch, warp_amd, synth, cfg, books, a.stack_tokens,
                            budget_gb=a.stack_budget_gb)
        log(f"[bench] stack {stack['tok_s']} tok/s, hit rate {stack['hit_rate']}")
        # the same stack and tokens with the lookahead's guesses inside the
        # next layer's group limit: a guess in a group the routing drops is
        # never selected, so its read is wasted
        if a.stack_grouped:
            v = bench_stack(torch, warp_amd, synth, cfg, books, a.stack_tokens, budget_gb=a.stack_budget_gb,
                            grouped=True)
            stack["lookahead_grouped"] = {k: v[k] for k in (
                "lookahead", "lookahead_rule", "hit_rate", "misses", "lookahead_reads", "lookahead_reads_used",
                "lookahead_reads_wasted", "gb_read", "gb_read_per_token", "tok_s", "ms_per_token",
                "tok_s_second_half", "host_to_device_gbps")}
            stack["lookahead_grouped"]["lookahead_precision_top6"] = v["routing"]["lookahead_precision_top6"]
            log(f"[bench] stack, grouped lookahead: {v['tok_s']} tok/s, hit rate {v['hit_rate']}, "
                f"{v['gb_read_per_token']} GB/token")

    cpu = None
    if not a.no_cpu and B == 1:
        host = host_cpu()
        # every physical core this process may use, within the host's share
        # of CPUs (OMP_NUM_THREADS where set; 16 otherwise)
        share = int(os.environ.get("OMP_NUM_THREADS", "0")) or 16
        nthreads = max(1, min(share, host["physical_cores_in_affinity"] or host["affinity_cpus"]))
        xs = x_all[a.warmup:].to(torch.float32).numpy()
        n, t_used, isa, n1, t1 = cpu_baseline(torch, cfg, slab, books, rb, trunk, xs, a.cpu_seconds, nthreads)
        cpu = {"value": round(t_used / n * 1e6, 1), "unit": "us/token", "cores": nthreads,
               "kind": "port",
               "sample": f"{n} tokens ({t_used:.1f} s) of the same {a.config} batch-1 layer, the timed "
                         f"steps' {len(xs)} tokens cycled, {isa} kernels, after one untimed warm-up token",
               "single_thread_value": round(t1 / n1 * 1e6, 1), "single_thread_sample": f"{n1} tokens ({t1:.1f} s)",
               "host": host}
        try:
            with open(os.path.join(ROOT, "tests", "golden", "cpu_calibration.json")) as f:
                cal = json.load(f)
            cpu["calibration"] = {
                "what": "restatement time / the reference engine's moe_layer compiled from its sources, "
                        "same layer, tokens and threads, outputs bit-exact",
                "host": cal["host"]["model"],
                "ratio_by_threads": {k: v["restatement_over_reference"] for k, v in cal["threads"].items()}}
        except (OSError, KeyError, ValueError):
            pass

    out = {
        "metric": METRIC,
        "value": us_per_token,
        "unit": "us/token",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights VQ3R-encoded on device; bf16 N(0,1) tokens)"
                if cfg["bf16"] else "synthetic (seeded N(0,0.02) weights VQ3R-encoded on device; "
                                    "fp32 N(0,1) tokens)",
        "config": {"workload": f"{a.config} MoE layer decode, batch {B}", "hidden": H,
                   "experts": E, "top_k": K, "moe_inter": I, "batch": B,
                   "layers_cycled": a.layers},
        "hbm_gbps": dec["hbm_gbps"],
        "hbm_frac": dec["hbm_frac"],
        "bytes_per_step": dec["bytes_per_step"],
        "distinct_experts_per_step": dec["distinct_experts_per_step"],
        "wall_ms_per_step": dec["wall_ms_per_step"],
        "stage_us": dec["stage_us"],
        "roofline": {"bound": "hbm", "kernel": dom["kernel"],
                     "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "launch_us": dom["launch_us"], "algorithmic_bytes": dom["algorithmic_bytes"]},
        "decode_configs": per_config,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "vq4p_rows": vq4p,
        "formats": formats,
        "expert_cache": stack,
    }
    print(json.dumps(out))
    for m in layers:
        m.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
