# SPDX-License-Identifier: Apache-2.0
"""Synthetic MoE layer data in WARP's container layout, built with numpy.

Small, fast and deterministic: random codebooks, random index streams,
random f16 row scales, and trunk tensors (router, bias, shared expert) in
F32 / Q8G / Q4G.  The byte layout is the container's (expert record:
[48 B header][gate idx][up idx][down idx][f16 scales], 4 KiB padded;
src/waste_format.h:98-130, docs/FORMAT.md:171-263; Q-format rows:
tools/convert.py:893-924).  Used by the CPU tests, the golden-vector
script and the GPU parity tests at small sizes.
"""
import struct
import zlib

import numpy as np

MAGIC_EXPERT = 0x50584557
MAGIC_CODEBOOK = 0x4B424357
FMT_F32, FMT_Q8G, FMT_Q4G, FMT_VQ3R, FMT_VQ2R, FMT_VQ4P = 0, 2, 3, 4, 5, 8
STAGES, ENTRIES, VEC_DIM, BLOCK = 3, 256, 8, 64


def block_indices(idx, M, N):
    """idx [M][N/8][b] u8 (b = 3 bytes a (row, position) in both VQ3R and
    VQ4P) -> [ceil(M/64)][N/8][64][b], zero-padded rows
    (tools/convert.py:777-792)."""
    nv = N // VEC_DIM
    nb = (M + BLOCK - 1) // BLOCK
    b = idx.shape[2]
    pad = np.zeros((nb * BLOCK, nv, b), np.uint8)
    pad[:M] = idx
    return pad.reshape(nb, BLOCK, nv, b).transpose(0, 2, 1, 3).copy()


def pack_p6(codes):
    """VQ4P: four 6-bit codes [..][4] -> three bytes [..][3], code s at bit
    6s of the little-endian 24-bit word (the inverse of the engine's
    P6_J0..P6_J3, src/simd.h:73-76)."""
    c = codes.astype(np.uint32)
    w = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)
    return np.stack([w & 0xFF, (w >> 8) & 0xFF, (w >> 16) & 0xFF], -1).astype(np.uint8)


def unblock_indices(raw, M, N):
    nv = N // VEC_DIM
    nb = (M + BLOCK - 1) // BLOCK
    t = np.frombuffer(raw, np.uint8, nb * nv * BLOCK * STAGES)
    return t.reshape(nb, nv, BLOCK, STAGES).transpose(0, 2, 1, 3).reshape(nb * BLOCK, nv, STAGES)[:M]


def make_record(layer, eid, cb_base, shapes, idx_list, scale_list, fmt=FMT_VQ3R):
    """One WEXP record.  shapes = [(I,H),(I,H),(H,I)]; idx_list[k] is
    [M][N/8][3] u8 (VQ3R codes, or VQ4P's packed bytes); scale_list[k] is
    [M] f16 bits (u16)."""
    body = bytearray()
    offs = []
    off = 48
    for (M, N), idx in zip(shapes, idx_list):
        offs.append(off)
        b = block_indices(idx, M, N).tobytes()
        body += b
        off += len(b)
    corr = off
    for s in scale_list:
        body += np.asarray(s, np.uint16).tobytes()
    total = 48 + len(body)
    blocks = (total + 4095) // 4096
    hdr = struct.pack("<IHHBBHHHIIIIIIII", MAGIC_EXPERT, layer, eid, fmt, 0,
                      cb_base, 0, 0, blocks, offs[0], offs[1], offs[2], corr,
                      zlib.crc32(bytes(body)) & 0xFFFFFFFF, 0, 0)
    rec = bytearray(blocks * 4096)
    rec[:48] = hdr
    rec[48:48 + len(body)] = body
    return bytes(rec)


from warp_amd.synth import Tensor, f16_bits, quant_q4g, quant_q8g  # noqa: E402,F401


class Layer:
    """One synthetic MoE layer.  index_bits 8: VQ3R experts (three stages
    of 256 entries), or VQ2R with stages=2 (two bytes a row and position);
    6: VQ4P (four stages of 64, the codes packed in three bytes); idx then
    holds the unpacked codes [M][N/8][4]."""

    def __init__(self, H, I, E, K, *, score_func=0, renorm=0, routed_scale=1.0,
                 n_group=1, topk_group=1, n_shared=0, router_fmt=FMT_F32,
                 shared_fmt=FMT_Q8G, bias=False, seed=0, cb_base=0,
                 book_scale=0.3, subnormal_books=0, layer=0, index_bits=8, stages=3):
        rng = np.random.default_rng(seed)
        self.H, self.I, self.E, self.K = H, I, E, K
        self.score_func, self.renorm, self.routed_scale = score_func, renorm, routed_scale
        self.n_group, self.topk_group, self.n_shared = n_group, topk_group, n_shared
        self.cb_base = cb_base
        self.layer = layer
        self.index_bits = index_bits
        self.stages, self.entries = (4, 64) if index_bits == 6 else (stages, ENTRIES)
        assert index_bits == 6 or stages in (2, 3)
        self.n_books = cb_base + 3 * self.stages
        books = (rng.standard_normal((self.n_books, self.entries, VEC_DIM)) * book_scale).astype(np.float32)
        self.books_f16 = f16_bits(books)
        if subnormal_books:
            # plant fp16 subnormals: the loader flushes them to signed zero
            flat = self.books_f16.reshape(-1)
            pos = rng.choice(flat.size, subnormal_books, replace=False)
            flat[pos] = (rng.integers(1, 1024, subnormal_books) |
                         (rng.integers(0, 2, subnormal_books) << 15)).astype(np.uint16)
        shapes = [(I, H), (I, H), (H, I)]
        self.shapes = shapes
        self.records = []
        self.idx = []
        self.scales = []
        for e in range(E):
            il = [rng.integers(0, self.entries, (M, N // VEC_DIM, self.stages), dtype=np.uint8)
                  for M, N in shapes]
            sl = [f16_bits(rng.uniform(0.01, 0.05, M)) for M, _ in shapes]
            self.idx.append(il)
            self.scales.append(sl)
            if index_bits == 6:
                self.records.append(make_record(layer, e, cb_base, shapes, [pack_p6(c) for c in il], sl,
                                                FMT_VQ4P))
            else:
                self.records.append(make_record(layer, e, cb_base, shapes, il, sl,
                                                FMT_VQ2R if self.stages == 2 else FMT_VQ3R))
        self.rec_bytes = len(self.records[0])
        self.router = Tensor.make(router_fmt, (rng.standard_normal((E, H)) * 0.02).astype(np.float32))
        self.bias = (rng.standard_normal(E) * 0.02).astype(np.float32) if bias else None
        SI = I * (n_shared if n_shared else 1)
        if n_shared:
            self.sh = [Tensor.make(shared_fmt, (rng.standard_normal((SI, H)) * 0.02).astype(np.float32)),
                       Tensor.make(shared_fmt, (rng.standard_normal((SI, H)) * 0.02).astype(np.float32)),
                       Tensor.make(shared_fmt, (rng.standard_normal((H, SI)) * 0.02).astype(np.float32))]
        else:
            self.sh = [Tensor.absent()] * 3
        self.rng = rng

    def bank(self):
        return b"".join(self.records)

    def inputs(self, T, seed=1):
        r = np.random.default_rng(seed)
        return r.standard_normal((T, self.H)).astype(np.float32)


def quant_q3g(W, group=128, codes=False):
    """Q3G rows (tools/convert.py:854-892): codes round(w/scale) in [-4, 3]
    biased by +4, LSB-first at bit 3i of the row, each row padded to
    (n*3+7)/8 bytes plus one guard byte; scale = amax/3 per group, f16.
    Returns (packed uint8 [rows][rowbytes], f16 scale bits [rows][ng],
    rowbytes), and with codes=True also the signed codes [rows][n]."""
    rows, N = W.shape
    ng = (N + group - 1) // group
    n = ng * group
    Wp = np.zeros((rows, n), np.float32)
    Wp[:, :N] = W
    g = Wp.reshape(rows, ng, group)
    sc = np.maximum(np.abs(g).max(-1, keepdims=True), np.float32(1e-8)) / np.float32(3.0)
    sc16 = sc.astype(np.float16)
    u = (np.clip(np.rint(g / sc), -4, 3).astype(np.int32) + 4).reshape(rows, n)
    rowbytes = (n * 3 + 7) // 8 + 1
    buf = np.zeros((rows, rowbytes), np.int32)
    off = np.arange(n) * 3
    byte, shift = off // 8, off % 8
    for i in range(n):
        buf[:, byte[i]] += (u[:, i] << shift[i]) & 0xFF
        if shift[i] > 5:
            buf[:, byte[i] + 1] += (u[:, i] >> (8 - shift[i])) & 0xFF
    out = (buf.astype(np.uint8), sc16.view(np.uint16).reshape(rows, ng), rowbytes)
    return out + (u - 4,) if codes else out
