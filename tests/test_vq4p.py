# SPDX-License-Identifier: Apache-2.0
"""VQ4P (6-bit codes, four stages of 64 entries) through the engine's int8
LUT: the oracle against the compiled reference's golden vectors and closed
forms (CPU), then the device kernels and the vq_rows_p6 slot against the
oracle, bit for bit (GPU).

  orc_vq_quant_lut  golden (src/model.c:3979-4074 compiled, both tables),
                    a planted table (an all-zero block, halves under a unit
                    inverse: ties to even), and the rounding bound
                    |lut - q*scale| <= scale/2
  orc_vq_rows_p6    golden in both fold orders (the portable C kernel and
                    the AVX-512 VBMI one), and the integer block sums
                    recomputed with numpy gathers from the unpacked codes
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from oracle_lib import Oracle, fp, i8p, ptr, u16p, u8p  # noqa: E402
from make_golden import vq4p_inputs  # noqa: E402

GOLD = os.path.join(HERE, "golden", "vq4p.npz")


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def unpack(idx, M, nv):
    """codes[r][v][s] from the blocked three-byte layout (src/simd.h:73-76)."""
    b = idx.reshape(M // 64, nv, 64, 3).astype(np.int64)
    b0, b1, b2 = b[..., 0], b[..., 1], b[..., 2]
    j = np.stack([b0 & 63, ((b0 >> 6) | (b1 << 2)) & 63, ((b1 >> 4) | (b2 << 4)) & 63, (b2 >> 2) & 63], -1)
    return j.transpose(0, 2, 1, 3).reshape(M, nv, 4)


def test_inputs_are_the_golden_ones(gold):
    import hashlib
    books16, _, x, idx, scale, qlut, _, _ = vq4p_inputs()
    h = hashlib.sha256()
    for a in (books16, x, idx, scale, qlut):
        h.update(a.tobytes())
    assert str(gold["digest"]) == h.hexdigest()


def test_quant_golden(orc, gold):
    _, _, _, _, _, qlut, M, nv = vq4p_inputs()
    for o in (0, 1):
        q, qs = orc.vq_quant_lut(gold[f"lut{o}"], nv)
        assert np.array_equal(q, gold[f"q{o}"]) and np.array_equal(bits(qs), bits(gold[f"qs{o}"]))
    q, qs = orc.vq_quant_lut(qlut, 64)
    assert np.array_equal(q, gold["qq"]) and np.array_equal(bits(qs), bits(gold["qsc"]))


def test_quant_planted(orc):
    _, _, _, _, _, qlut, _, _ = vq4p_inputs()
    q, qs = orc.vq_quant_lut(qlut, 64)
    q = q.reshape(64, 256)
    assert qs[0] == 0.0 and not q[:32].any()                      # all-zero block
    assert qs[1] == 1.0                                          # max 127: inverse 1
    assert q[32, :8].tolist() == [0, 2, 2, 0, -2, -2, 126, -126]  # halves to even


def test_quant_bound(orc, gold):
    lut = gold["lut1"].reshape(-1).astype(np.float64)
    q, qs = orc.vq_quant_lut(gold["lut1"], 80)
    blk = np.repeat(np.arange(3), 32 * 256)[:lut.size]
    s = qs[blk].astype(np.float64)
    assert np.abs(q).max() <= 127
    assert np.all(np.abs(lut - q * s) <= 0.5 * s * (1 + 1e-6) + 1e-30)


def test_rows_golden(orc, gold):
    _, _, _, idx, scale, _, M, nv = vq4p_inputs()
    for o in (0, 1):
        y = orc.vq_rows_p6(idx, scale, gold[f"q{o}"], gold[f"qs{o}"], M, nv, o)
        assert np.array_equal(bits(y), bits(gold[f"rows{o}"])), o
    # the two fold orders are told apart by these inputs
    assert not np.array_equal(bits(gold["rows0"]), bits(gold["rows1"]))


def test_rows_integer_sums(orc, gold):
    """The block sums recomputed from the unpacked codes with numpy, folded
    both ways in fp32, equal the oracle's rows."""
    _, _, _, idx, scale, _, M, nv = vq4p_inputs()
    j = unpack(idx, M, nv)
    for o in (0, 1):
        T = gold[f"q{o}"].reshape(nv, 4, 64).astype(np.int64)
        ent = T[np.arange(nv)[None, :, None], np.arange(4)[None, None, :], j]     # [M][nv][4]
        per_v = ent.sum(-1)
        sums = np.stack([per_v[:, b:b + 32].sum(1) for b in range(0, nv, 32)], 1)  # [M][3]
        ls = gold[f"qs{o}"]
        acc = np.zeros(M, np.float32)
        for b in range(sums.shape[1]):
            prod = (np.float64(ls[b]) * sums[:, b].astype(np.float64))
            if o == 0:
                acc = (acc + prod.astype(np.float32)).astype(np.float32)
            else:                                  # one rounding of acc + ls*sum
                acc = (acc.astype(np.float64) + prod).astype(np.float32)
        sc = scale.view(np.float16).astype(np.float32)
        y = (acc * sc).astype(np.float32)
        ref = orc.vq_rows_p6(idx, scale, gold[f"q{o}"], gold[f"qs{o}"], M, nv, o)
        assert np.array_equal(bits(y), bits(ref)), o


# ---- the device kernels and the slot (MI355X) -----------------------------------

def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import warp_amd
    return torch, warp_amd.lib()


@pytest.mark.gpu
def test_device_quant_and_rows_bit_exact(orc, gold):
    torch, lib = _gpu()
    dev = torch.device("cuda:0")
    _, _, _, idx, scale, qlut, M, nv = vq4p_inputs()
    lib.waste_hip_vq_quant_lut.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    lib.waste_hip_vq_rows_p6.argtypes = [C.c_void_p] * 4 + [C.c_int] * 4 + [C.c_void_p, C.c_void_p]
    s = torch.cuda.current_stream().cuda_stream
    for tab, nvq in ((gold["lut0"], nv), (gold["lut1"], nv), (qlut, 64)):
        d = torch.from_numpy(np.ascontiguousarray(tab, np.float32).reshape(-1)).to(dev)
        q = torch.zeros(d.numel(), dtype=torch.int8, device=dev)
        qs = torch.zeros((nvq + 31) // 32, dtype=torch.float32, device=dev)
        assert lib.waste_hip_vq_quant_lut(d.data_ptr(), nvq, 4, 64, q.data_ptr(), qs.data_ptr(), s) == 0
        torch.cuda.synchronize()
        q_ref, qs_ref = orc.vq_quant_lut(tab, nvq)
        assert np.array_equal(q.cpu().numpy(), q_ref)
        assert np.array_equal(bits(qs.cpu().numpy()), bits(qs_ref))
    di = torch.from_numpy(idx).to(dev)
    ds = torch.from_numpy(scale.view(np.int16)).to(dev)
    for o in (0, 1):
        dq = torch.from_numpy(gold[f"q{o}"]).to(dev)
        dls = torch.from_numpy(gold[f"qs{o}"]).to(dev)
        for lo, hi in ((0, M), (64, M), (0, 100), (128, 150)):
            y = torch.full((M,), float("nan"), device=dev)
            assert lib.waste_hip_vq_rows_p6(di.data_ptr(), ds.data_ptr(), dq.data_ptr(), dls.data_ptr(),
                                            lo, hi, nv, o, y.data_ptr(), s) == 0
            torch.cuda.synchronize()
            yh = y.cpu().numpy()
            ref = orc.vq_rows_p6(idx, scale, gold[f"q{o}"], gold[f"qs{o}"], M, nv, o)
            assert np.array_equal(bits(yh[lo:hi]), bits(ref[lo:hi])), (o, lo, hi)
            assert np.isnan(yh[:lo]).all() and np.isnan(yh[hi:]).all()


@pytest.mark.gpu
def test_slot_rows_bit_exact(orc, gold):
    """waste_register_hip's vq_rows_p6 slot (waste_kernels offset 40,
    src/waste_backend.h:85), installed only with WASTE_HIP_P6=1, on host
    buffers, over the ranges the engine's pool hands it, against the CPU
    kernel of this host's fold order."""
    torch, lib = _gpu()
    _, _, _, idx, scale, _, M, nv = vq4p_inputs()
    lib.waste_register_hip.restype = C.c_char_p
    sentinel = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)(lambda b, e, p: None)
    tab = (C.c_uint8 * 80)()
    C.cast(C.addressof(tab) + 40, C.POINTER(C.c_void_p))[0] = C.cast(sentinel, C.c_void_p).value
    os.environ.pop("WASTE_HIP_P6", None)
    assert lib.waste_register_hip(C.cast(tab, C.c_void_p))
    # not asked for: the CPU kernel the table held stays in the slot
    assert C.cast(C.addressof(tab) + 40, C.POINTER(C.c_void_p)).contents.value == C.cast(sentinel, C.c_void_p).value
    tab = (C.c_uint8 * 80)()
    os.environ["WASTE_HIP_P6"] = "1"
    try:
        assert lib.waste_register_hip(C.cast(tab, C.c_void_p))
    finally:
        os.environ.pop("WASTE_HIP_P6", None)
    fnp = C.cast(C.addressof(tab) + 40, C.POINTER(C.c_void_p)).contents.value
    assert fnp
    slot = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)(fnp)

    class VqpArg(C.Structure):        # src/simd.h:57-61
        _fields_ = [("y", C.c_void_p), ("idx", C.c_void_p), ("scale", C.c_void_p), ("lut8", C.c_void_p),
                    ("lscale", C.c_void_p), ("nv", C.c_int)]
    order = lib.waste_hip_vq_p6_order()
    q, qs = gold[f"q{order}"], gold[f"qs{order}"]
    y = np.full(M, np.nan, np.float32)
    a = VqpArg(y.ctypes.data, idx.ctypes.data, scale.ctypes.data, q.ctypes.data, qs.ctypes.data, nv)
    for lo, hi in ((0, 64), (64, 192)):
        slot(lo, hi, C.cast(C.pointer(a), C.c_void_p))
    assert np.array_equal(bits(y), bits(gold[f"rows{order}"]))
    # a 150-row matrix: its last block partial, the index buffer ending at
    # that block's last row (the slot copies no byte past it)
    Mp = 150
    idxp = np.ascontiguousarray(idx[:((Mp // 64) * nv + nv - 1) * 192 + (Mp % 64) * 3])
    scp = np.ascontiguousarray(scale[:Mp])
    y = np.full(Mp, np.nan, np.float32)
    a = VqpArg(y.ctypes.data, idxp.ctypes.data, scp.ctypes.data, q.ctypes.data, qs.ctypes.data, nv)
    for lo, hi in ((0, 128), (128, Mp)):
        slot(lo, hi, C.cast(C.pointer(a), C.c_void_p))
    assert np.array_equal(bits(y), bits(gold[f"rows{order}"][:Mp]))
