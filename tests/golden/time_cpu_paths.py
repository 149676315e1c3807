# SPDX-License-Identifier: Apache-2.0
"""Times the CPU baseline's restatement (liboracle.so, orc_moe_layer_mt)
against the reference engine's own moe_layer compiled from its sources
(oracle/_ref/libwasteref.so, ref_moe_time) on one DeepSeek-V3-shaped layer,
the same tokens, the same thread counts, and writes the ratio to
tests/golden/cpu_calibration.json.

    PYTHONPATH=/root/repo:/root/repo/tests python tests/golden/time_cpu_paths.py [--tokens 24]

Both sides run with every routed record resident in host memory (the
reference through an expert cache that holds the bank, filled by one
untimed pass over the tokens; the restatement reads the records in place)
and split each matrix's rows over a pool of the given size.  The layer is
the decode benchmark's shape (hidden 7168, 256 experts of width 2048,
sigmoid + bias, top-8 renormalised, scale 2.5, one 4-bit shared expert, F32
router) with ungrouped routing: the reference has no group-limited top-k,
and which 8 experts a token picks does not change the work.  The last
token's outputs of the two are compared bit for bit.
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle_lib import Oracle, Ref, _OrcLayer  # noqa: E402
from records import FMT_F32, FMT_Q4G, Layer  # noqa: E402
from bench import host_cpu  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=24)
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--threads", default="1,8")
    ap.add_argument("--out", default=os.path.join(HERE, "cpu_calibration.json"))
    a = ap.parse_args()
    t0 = time.time()
    L = Layer(7168, 2048, 256, 8, score_func=0, renorm=1, routed_scale=2.5, n_shared=1,
              router_fmt=FMT_F32, shared_fmt=FMT_Q4G, bias=True, seed=0)
    L.idx = None                                 # the unblocked copies; only the records are read
    print(f"layer built in {time.time() - t0:.0f} s", flush=True)
    orc, ref = Oracle(), Ref()
    ref.set_order(1)
    if ref.isa != 2:
        print("this host does not run the reference's AVX-512 kernels", file=sys.stderr)
        return 1
    ol = _OrcLayer(orc, L, 1)
    bank = np.frombuffer(L.bank(), np.uint8)
    X = L.inputs(a.tokens, seed=5)
    res = {"layer": "dsv3 shape, ungrouped routing, seed 0", "tokens": a.tokens, "repeats": a.repeats,
           "isa": "AVX-512", "host": host_cpu(), "threads": {}}
    for nt in [int(t) for t in a.threads.split(",")]:
        t_orc, t_ref = [], []
        for _ in range(a.repeats):
            for x in X:                               # warm: caches and the thread pool
                ol.layer_mt(x, nt)
            s0 = time.perf_counter()
            for x in X:
                rc, out_o, _, _ = ol.layer_mt(x, nt)
            t_orc.append(time.perf_counter() - s0)
            sec, out_r = ref.moe_time(L, X, ol.booksT, nt, bank=bank)
            if sec < 0:
                print(f"ref_moe_time failed: {sec}", file=sys.stderr)
                return 1
            t_ref.append(sec)
        mo, mr = statistics.median(t_orc), statistics.median(t_ref)
        same = bool(np.array_equal(out_o.view(np.uint32), out_r.view(np.uint32)))
        res["threads"][str(nt)] = {
            "restatement_us_per_token": round(mo / a.tokens * 1e6, 1),
            "reference_us_per_token": round(mr / a.tokens * 1e6, 1),
            "restatement_over_reference": round(mo / mr, 3),
            "last_token_bit_exact": same,
            "samples_s": {"restatement": [round(t, 4) for t in t_orc], "reference": [round(t, 4) for t in t_ref]}}
        print(nt, res["threads"][str(nt)], flush=True)
    with open(a.out, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
