# SPDX-License-Identifier: Apache-2.0
"""Helpers for the GPU tests: build a device layer from a records.Layer and
compare it with the oracle."""
import numpy as np

import warp_amd

# The tolerance for layer outputs: max relative error 1e-3 with
# fp32 accumulation, measured normwise (max |y - ref| / max |ref|).
LAYER_RTOL = 1e-3
# Router logits are an fp32 GEMV in a different summation order.
LOGIT_RTOL = 1e-5


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def gpu_layer(L, max_tokens=1, verify=0, prefill_min=0, records=True, p6_order=None):
    m = warp_amd.MoeLayer(hidden=L.H, n_experts=L.E, top_k=L.K, moe_inter=L.I,
                          n_shared=L.n_shared, score_func=L.score_func, renorm=L.renorm,
                          routed_scale=L.routed_scale, n_group=L.n_group,
                          topk_group=L.topk_group, layer=getattr(L, "layer", 0),
                          max_tokens=max_tokens, verify_records=verify,
                          prefill_min_tokens=prefill_min, index_bits=getattr(L, "index_bits", 8),
                          p6_order=p6_order, stages=getattr(L, "stages", 0))
    m.set_codebooks(L.books_f16)
    m.set_router(L.router, L.bias)
    if L.n_shared:
        m.set_shared(*L.sh)
    if records:
        for e, rec in enumerate(L.records):
            rc = m.set_expert(e, rec)
            assert rc == 0, (e, rc)
    return m


def run_forward(torch, m, L, X, bf16=False):
    """X [T][H] float32 numpy (already bf16-representable when bf16)."""
    T = X.shape[0]
    dev = torch.device("cuda:0")
    if bf16:
        xd = torch.from_numpy(X).to(dev).to(torch.bfloat16)
    else:
        xd = torch.from_numpy(X).to(dev)
    y = torch.empty((T, L.H), dtype=torch.float32, device=dev)
    ids = torch.empty((T, L.K), dtype=torch.int32, device=dev)
    w = torch.empty((T, L.K), dtype=torch.float32, device=dev)
    lg = torch.empty((T, L.E), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    m.forward(xd.data_ptr(), T, y.data_ptr(), ids.data_ptr(), w.data_ptr(), lg.data_ptr(),
              bf16=bf16, stream=s)
    st = m.status(s)
    return st, y.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), lg.cpu().numpy()
