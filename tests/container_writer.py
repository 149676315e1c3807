# SPDX-License-Identifier: Apache-2.0
"""Writes a WARP container directory from records.Layer objects: the
container reader's test fixture, in the reference's on-disk format.

Files and keys (docs/FORMAT.md:54-101): manifest.json with format_version
0, tensor_prefix, config (the release's own keys), expert_quant, layers
(file, experts, bytes, codebook_base) and trunk (name, fmt, off, shape,
group, scale_off, bytes); trunk.bin with each tensor's payload at `off`
(F32 rows, or Q rows with their f16 group scales at `scale_off`;
src/model.c:1366-1395); codebooks.bin as 16-byte headers each followed by
256 x 8 fp16 (src/waste_format.h:139-150); experts-L<n>.bin as the layer's
4 KiB records in expert order (src/waste_format.h:98-132).

Every MoE layer takes 3 x stages books of its own (nine for VQ3R, twelve
for VQ4P, six for VQ2R), codebook_base = that count x its rank among the MoE layers, so
each records.Layer must be built with that cb_base and with layer = its
index.  The layers' format (VQ3R; VQ2R: two stages; or VQ4P: index_bits 6,
four stages of 64 entries) is the container's expert_quant, as tools/convert.py:2482-2488
writes it.
"""
import json
import os
import struct
import types

import numpy as np

from records import ENTRIES, FMT_F32, MAGIC_CODEBOOK, STAGES, VEC_DIM

SCORE_NAMES = {0: "sigmoid", 1: "softmax", 2: "sqrtsoftplus"}


class _Trunk:
    def __init__(self):
        self.buf = bytearray()
        self.index = []

    def _put(self, b):
        while len(self.buf) % 64:
            self.buf.append(0)
        off = len(self.buf)
        self.buf += b
        return off

    def f32(self, name, a, shape=None):
        a = np.ascontiguousarray(a, np.float32)
        off = self._put(a.tobytes())
        self.index.append({"name": name, "fmt": FMT_F32, "off": off,
                           "shape": list(shape or a.shape), "bytes": a.nbytes})

    def tensor(self, name, t):
        """A synth.Tensor (F32, Q8G or Q4G rows)."""
        if t.fmt == FMT_F32:
            self.f32(name, t.q, [t.rows, t.cols])
            return
        q = np.ascontiguousarray(t.q).view(np.uint8).tobytes()
        off = self._put(q)
        soff = self._put(np.ascontiguousarray(t.qs, np.uint16).tobytes())
        self.index.append({"name": name, "fmt": int(t.fmt), "off": off, "shape": [t.rows, t.cols],
                           "group": int(t.group), "scale_off": soff,
                           "bytes": len(q) + t.qs.size * 2})


def moe_names(prefix, L):
    p = f"{prefix}model.layers.{L}.block_sparse_moe."
    return {"router": p + "gate.weight", "bias": p + "gate.e_score_correction_bias",
            "gate": p + "shared_experts.gate_proj.weight", "up": p + "shared_experts.up_proj.weight",
            "down": p + "shared_experts.down_proj.weight"}


def build(layers, *, n_layers, first_dense, prefix="", text_config=False, vocab=1000):
    """The container as (manifest dict, {file name: bytes}) from MoE layers
    first_dense .. first_dense + len(layers) - 1."""
    L0 = layers[0]
    cfg = {"num_hidden_layers": n_layers, "hidden_size": L0.H, "vocab_size": vocab,
           "num_attention_heads": 8, "rms_norm_eps": 1e-6, "num_experts": L0.E,
           "num_experts_per_token": L0.K, "moe_intermediate_size": L0.I,
           "num_shared_experts": L0.n_shared, "first_k_dense_replace": first_dense,
           "routed_scaling_factor": L0.routed_scale, "scoring_func": SCORE_NAMES[L0.score_func],
           "n_group": L0.n_group, "topk_group": L0.topk_group}
    if L0.renorm:
        cfg["moe_renormalize"] = True
    trunk = _Trunk()
    trunk.f32(f"{prefix}model.norm.weight", np.ones(L0.H, np.float32))
    files, bank_index, books = {}, {}, []
    st, en, ib = getattr(L0, "stages", STAGES), getattr(L0, "entries", ENTRIES), getattr(L0, "index_bits", 8)
    nbk = 3 * st
    for rank, Lyr in enumerate(layers):
        L = first_dense + rank
        assert Lyr.layer == L and Lyr.cb_base == nbk * rank, "build each layer with its index and cb_base"
        assert getattr(Lyr, "index_bits", 8) == ib, "one expert format per container"
        n = moe_names(prefix, L)
        trunk.tensor(n["router"], Lyr.router)
        if Lyr.bias is not None:
            trunk.f32(n["bias"], Lyr.bias)
        for k, t in zip(("gate", "up", "down"), Lyr.sh):
            trunk.tensor(n[k], t)
        name = f"experts-L{L}.bin"
        files[name] = Lyr.bank()
        bank_index[str(L)] = {"file": name, "experts": Lyr.E, "bytes": len(files[name]),
                              "codebook_base": Lyr.cb_base}
        books.append(Lyr.books_f16[Lyr.cb_base:Lyr.cb_base + nbk])
    cb = bytearray()
    for cid, book in enumerate(np.concatenate(books)):
        # the converter writes FMT_VQ3R in every codebook header
        # (tools/convert.py:1298-1302), whatever the layers' format
        cb += struct.pack("<IHBBII", MAGIC_CODEBOOK, cid & 0xFFFF, 4, VEC_DIM, en, 0)
        cb += np.ascontiguousarray(book, np.uint16).tobytes()
    files["codebooks.bin"] = bytes(cb)
    files["trunk.bin"] = bytes(trunk.buf)
    manifest = {"format_version": 0, "arch": "synthetic", "tensor_prefix": prefix,
                "config": {"text_config": cfg} if text_config else cfg,
                "expert_quant": {"fmt": "VQ3R", "stages": STAGES, "vec_dim": VEC_DIM,
                                 "entries": ENTRIES, "index_block": 64, "bits_per_weight": STAGES},
                "layers": bank_index, "trunk": trunk.index}
    if ib == 6:
        manifest["expert_quant"] = {"fmt": "VQ4P", "stages": st, "vec_dim": VEC_DIM, "entries": en,
                                    "index_block": 64, "index_bits": 6, "bits_per_weight": st * 6 / VEC_DIM}
    elif st == 2:
        manifest["expert_quant"] = {"fmt": "VQ2R", "stages": 2, "vec_dim": VEC_DIM, "entries": en,
                                    "index_block": 64, "index_bits": 8, "bits_per_weight": 2}
    if text_config and prefix == "language_model.":
        manifest["tensor_prefix"] = ""            # the reader supplies it for a nested config
    return manifest, files


def write(path, manifest, files):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    for name, data in files.items():
        with open(os.path.join(path, name), "wb") as f:
            f.write(data)
    return path


def oracle_view(c, layer, group_limit=False):
    """What a warp_amd.Container holds for one MoE layer, as the attributes
    the oracle's layer takes (oracle_lib.Oracle.moe): built from the
    reader's output alone."""
    g = c.config()
    n, cb, rb = c.bank(layer)
    p = f"{g['prefix']}model.layers.{layer}.block_sparse_moe."
    recs = []
    for e in range(n):
        rc, r = c.read_expert(layer, e)
        assert rc == 0, (layer, e, rc)
        recs.append(r.tobytes())
    try:
        bias = np.ascontiguousarray(c.tensor(p + "gate.e_score_correction_bias").q.reshape(-1), np.float32)
    except Exception:
        bias = None
    books = c.codebooks()
    return types.SimpleNamespace(
        H=g["hidden"], I=g["moe_inter"], E=g["n_experts"], K=g["top_k"], n_shared=max(g["n_shared"], 1),
        score_func=g["score_func"], renorm=g["renorm"], routed_scale=g["routed_scale"],
        n_group=g["n_group"] if group_limit else 1, topk_group=g["topk_group"] if group_limit else 1,
        books_f16=books, n_books=books.shape[0], records=recs, rec_bytes=rb, cb_base=cb, layer=layer,
        router=c.tensor(p + "gate.weight"), bias=bias,
        sh=[c.tensor(p + "shared_experts." + k + "_proj.weight") for k in ("gate", "up", "down")])
