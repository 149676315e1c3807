# SPDX-License-Identifier: Apache-2.0
"""The container reader on the CPU: round trips through the repo's own
writer, the engine's refusals, record checks and crc32.

crc32 known answers are the reference suite's zlib values
(tests/test_container.c:35-73).  Refusals follow the checks of
waste_model_open and record_check (src/model.c:2640-2741, 2957-3100,
3645-3692) and load_trunk (src/model.c:1306-1330); each case mutates one
field of a container that otherwise opens.
"""
import copy
import ctypes
import json
import os
import struct
import subprocess
import zlib

import numpy as np
import pytest

import warp_amd
from container_writer import build, moe_names, oracle_view, write
from oracle_lib import Oracle
from records import FMT_F32, FMT_Q4G, FMT_Q8G, Layer

H, I, E, K = 256, 128, 8, 2


def layers(n=2, first_dense=1, **kw):
    base = dict(score_func=0, renorm=1, routed_scale=2.5, bias=True, n_shared=1, shared_fmt=FMT_Q4G,
                router_fmt=FMT_F32)
    base.update(kw)
    return [Layer(H, I, E, K, seed=100 + r, cb_base=9 * r, layer=first_dense + r, **base) for r in range(n)]


@pytest.fixture(scope="module")
def fixture():
    Ls = layers()
    manifest, files = build(Ls, n_layers=3, first_dense=1)
    return Ls, manifest, files


def make(tmp_path, manifest, files, name="c"):
    return write(str(tmp_path / name), manifest, files)


def opened(path, verify=False):
    h = warp_amd.lib()
    out = __import__("ctypes").c_void_p()
    rc = h.waste_hip_container_open(os.fsencode(path), int(verify), __import__("ctypes").byref(out))
    if rc == 0:
        h.waste_hip_container_close(out)
    return rc


# ---- crc32 -------------------------------------------------------------

def test_crc32_known_answers():
    for s, want in [(b"", 0x00000000), (b"a", 0xE8B7BE43), (b"123456789", 0xCBF43926),
                    (b"The quick brown fox jumps over the lazy dog", 0x414FA339)]:
        assert warp_amd.crc32(s) == want == zlib.crc32(s)
    i = np.arange(65536, dtype=np.int64)
    buf = ((i * 31 + (i >> 11)) & 0xFF).astype(np.uint8)
    for off, n, want in [(0, 65536, 0x857C6B4F), (0, 3071, 0xE08F605E), (0, 3073, 0x331C420A),
                         (3, 40001, 0x5BBC9F51), (7, 65529, 0xB1F5AE9A)]:
        part = np.ascontiguousarray(buf[off:off + n])
        assert warp_amd.crc32(part) == want == zlib.crc32(part.tobytes())
    # a running value continues a split buffer
    a = warp_amd.crc32(buf[:1000])
    assert warp_amd.crc32(np.ascontiguousarray(buf[1000:5000]), a) == zlib.crc32(buf[:5000].tobytes())


# ---- round trip --------------------------------------------------------

@pytest.mark.parametrize("prefix,nested", [("", False), ("language_model.", False),
                                           ("language_model.", True)])
def test_round_trip(tmp_path, prefix, nested):
    Ls = layers(score_func=1, renorm=0, routed_scale=1.0, shared_fmt=FMT_Q8G) if nested else layers()
    manifest, files = build(Ls, n_layers=3, first_dense=1, prefix=prefix, text_config=nested)
    c = warp_amd.Container(make(tmp_path, manifest, files), verify=True)
    cfg = c.config()
    L0 = Ls[0]
    assert (cfg["n_layers"], cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]) == (3, H, E, K, I)
    assert (cfg["n_shared"], cfg["first_dense"], cfg["latent_dim"]) == (1, 1, 0)
    assert (cfg["score_func"], cfg["renorm"]) == (L0.score_func, L0.renorm)
    assert cfg["routed_scale"] == np.float32(L0.routed_scale)
    assert (cfg["stages"], cfg["vec_dim"], cfg["entries"], cfg["index_bits"], cfg["index_block"]) == (3, 8, 256, 8, 64)
    assert cfg["n_books"] == 18 and cfg["prefix"] == prefix
    assert c.bank(0) is None
    books = c.codebooks()
    for r, Lyr in enumerate(Ls):
        L = 1 + r
        n, cb, rb = c.bank(L)
        assert (n, cb, rb) == (E, 9 * r, Lyr.rec_bytes)
        assert np.array_equal(books[cb:cb + 9], Lyr.books_f16[cb:cb + 9])
        for e in range(E):
            rc, rec = c.read_expert(L, e)
            assert rc == 0 and rec.tobytes() == Lyr.records[e]
        dst = np.zeros((E, rb), np.uint8)
        assert c.read_bank(L, dst) == 0 and dst.tobytes() == Lyr.bank()
        names = moe_names(prefix, L)
        t = c.tensor(names["router"])
        assert t.fmt == Lyr.router.fmt and t.shape == (E, H)
        assert np.array_equal(t.q, Lyr.router.q)
        b = c.tensor(names["bias"])
        assert b.shape == (E,) and np.array_equal(b.q.reshape(-1), Lyr.bias)
        for k, ref in zip(("gate", "up", "down"), Lyr.sh):
            t = c.tensor(names[k])
            assert (t.fmt, t.rows, t.cols, t.group, t.rowbytes) == (ref.fmt, ref.rows, ref.cols, ref.group,
                                                                    ref.rowbytes)
            assert np.array_equal(t.q.view(np.int8), np.asarray(ref.q).view(np.int8).reshape(t.q.shape))
            assert np.array_equal(t.qs, ref.qs)
    assert c.error() == (0, 0, 0)
    with pytest.raises(warp_amd.HipError, match="EFORMAT"):
        c.tensor("model.layers.1.block_sparse_moe.no_such.weight")
    c.close()


def test_config_keys(tmp_path, fixture):
    """Alternate spellings and defaults, as cfg_from_json reads them
    (src/model.c:2186-2214)."""
    Ls, manifest, files = fixture
    m = copy.deepcopy(manifest)
    cfg = m["config"]
    cfg["num_experts_per_tok"] = cfg.pop("num_experts_per_token")
    del cfg["scoring_func"], cfg["routed_scaling_factor"], cfg["n_group"], cfg["topk_group"]
    cfg["moe_renormalize"] = False                  # presence is what counts
    del m["expert_quant"]                           # 3 stages x 256 x 8, index_bits 8
    c = warp_amd.Container(make(tmp_path, m, files))
    g = c.config()
    assert (g["top_k"], g["score_func"], g["routed_scale"], g["renorm"]) == (K, 0, 1.0, 1)
    assert (g["n_group"], g["topk_group"], g["stages"], g["entries"], g["vec_dim"]) == (1, 1, 3, 256, 8)
    cfg["scoring_func"] = "sqrtsoftplus"
    assert warp_amd.Container(make(tmp_path, m, files, "d")).config()["score_func"] == 2


# ---- refusals ----------------------------------------------------------

def _mut(manifest, f):
    m = copy.deepcopy(manifest)
    f(m)
    return m


MANIFEST_REFUSALS = {
    "no_version": lambda m: m.pop("format_version"),
    "version_1": lambda m: m.update(format_version=1),
    "version_str": lambda m: m.update(format_version="0"),
    "no_config": lambda m: m.pop("config"),
    "layers_0": lambda m: m["config"].update(num_hidden_layers=0),
    "layers_129": lambda m: m["config"].update(num_hidden_layers=129),
    "hidden_0": lambda m: m["config"].update(hidden_size=0),
    "vocab_missing": lambda m: m["config"].pop("vocab_size"),
    "heads_missing": lambda m: m["config"].pop("num_attention_heads"),
    "eps_1": lambda m: m["config"].update(rms_norm_eps=1.0),
    "topk_over_E": lambda m: m["config"].update(num_experts_per_token=E + 1),
    "topk_65": lambda m: m["config"].update(num_experts=128, num_experts_per_token=65),
    "topk_0": lambda m: m["config"].update(num_experts_per_token=0),
    "shared_65": lambda m: m["config"].update(num_shared_experts=65),
    "first_dense_over": lambda m: m["config"].update(first_k_dense_replace=4),
    "inter_neg": lambda m: m["config"].update(moe_intermediate_size=-1),
    "stages_0": lambda m: m["expert_quant"].update(stages=0),
    "stages_9": lambda m: m["expert_quant"].update(stages=9),
    "vec_dim_0": lambda m: m["expert_quant"].update(vec_dim=0),
    "vec_dim_65": lambda m: m["expert_quant"].update(vec_dim=65),
    "entries_257": lambda m: m["expert_quant"].update(entries=257),
    "index_bits_7": lambda m: m["expert_quant"].update(index_bits=7),
    "index_bits_6_vq3": lambda m: m["expert_quant"].update(index_bits=6),
    "index_block_32": lambda m: m["expert_quant"].update(index_block=32),
    "index_block_0": lambda m: m["expert_quant"].update(index_block=0),
    "bank_missing": lambda m: m["layers"].pop("2"),
    "bank_on_dense": lambda m: m["layers"].update({"0": dict(m["layers"]["1"])}),
    "experts_mismatch": lambda m: m["layers"]["1"].update(experts=E - 1),
    "bytes_ragged": lambda m: m["layers"]["1"].update(bytes=m["layers"]["1"]["bytes"] - 1),
    "bytes_0": lambda m: m["layers"]["1"].update(bytes=0),
    "cb_base_neg": lambda m: m["layers"]["1"].update(codebook_base=-1),
    "cb_base_over": lambda m: m["layers"]["2"].update(codebook_base=10),
    "file_parent": lambda m: m["layers"]["1"].update(file="../experts-L1.bin"),
    "file_absolute": lambda m: m["layers"]["1"].update(file="/etc/passwd"),
    "file_empty": lambda m: m["layers"]["1"].update(file=""),
    "trunk_not_list": lambda m: m.update(trunk={}),
    "shape_empty": lambda m: m["trunk"][1].update(shape=[]),
    "shape_zero": lambda m: m["trunk"][1].update(shape=[0, H]),
    "shape_5d": lambda m: m["trunk"][1].update(shape=[1, 1, 1, E, H]),
    "shape_huge": lambda m: m["trunk"][1].update(shape=[1 << 20, 1 << 20]),
    "group_0": lambda m: m["trunk"][3].update(group=0),
    "off_past_end": lambda m: m["trunk"][1].update(off=1 << 40),
    "off_neg": lambda m: m["trunk"][1].update(off=-64),
    "scale_off_past_end": lambda m: m["trunk"][3].update(scale_off=1 << 40),
    "name_too_long": lambda m: m["trunk"][1].update(name="x" * 600),
}


@pytest.mark.parametrize("case", sorted(MANIFEST_REFUSALS))
def test_manifest_refusals(tmp_path, fixture, case):
    Ls, manifest, files = fixture
    assert opened(make(tmp_path, manifest, files, "ok")) == 0
    m = _mut(manifest, MANIFEST_REFUSALS[case])
    assert opened(make(tmp_path, m, files, "bad")) == warp_amd.EFORMAT


def test_malformed_json(tmp_path, fixture):
    Ls, manifest, files = fixture
    path = make(tmp_path, manifest, files)
    text = open(os.path.join(path, "manifest.json")).read()
    for bad in [text[:len(text) // 2], text + "}", text.replace(":", "", 1), "[" + text + "]",
                text.replace('"format_version": 0', '"format_version": 0,'), "", "null"]:
        with open(os.path.join(path, "manifest.json"), "w") as f:
            f.write(bad)
        assert opened(path) == warp_amd.EFORMAT, bad[:40]


def test_missing_files(tmp_path, fixture):
    Ls, manifest, files = fixture
    for name in ("trunk.bin", "codebooks.bin", "experts-L1.bin", "manifest.json"):
        path = make(tmp_path, manifest, files, name)
        os.remove(os.path.join(path, name))
        assert opened(path) == warp_amd.EIO, name


def test_bank_short_by_a_record(tmp_path, fixture):
    """The probe of the last record (src/model.c:3089-3100): a bank missing
    whole records is refused at open; one cut inside its last record opens
    and fails that record's read."""
    Ls, manifest, files = fixture
    rb = Ls[0].rec_bytes
    f = dict(files)
    f["experts-L1.bin"] = files["experts-L1.bin"][:-rb]
    assert opened(make(tmp_path, manifest, f, "a")) == warp_amd.EIO
    f["experts-L1.bin"] = files["experts-L1.bin"][:-rb + 4096]
    c = warp_amd.Container(make(tmp_path, manifest, f, "b"))
    assert c.read_expert(1, E - 2)[0] == 0
    assert c.read_expert(1, E - 1)[0] == warp_amd.EIO
    assert c.error() == (warp_amd.EIO, 1, E - 1)


def test_tensor_extent(tmp_path, fixture):
    """A tensor whose payload runs past trunk.bin opens (the manifest's
    offsets are inside the file) and is refused when read."""
    Ls, manifest, files = fixture
    m = copy.deepcopy(manifest)
    size = len(files["trunk.bin"])
    router = next(t for t in m["trunk"] if t["name"].endswith("1.block_sparse_moe.gate.weight"))
    router["off"] = size - 16
    c = warp_amd.Container(make(tmp_path, m, files))
    with pytest.raises(warp_amd.HipError, match="EFORMAT"):
        c.tensor(router["name"])
    q = next(t for t in m["trunk"] if t["name"].endswith("1.block_sparse_moe.shared_experts.gate_proj.weight"))
    q["scale_off"] = size - 2
    c = warp_amd.Container(make(tmp_path, m, files, "d"))
    with pytest.raises(warp_amd.HipError, match="EFORMAT"):
        c.tensor(q["name"])


# ---- records -----------------------------------------------------------

def _patch(rec, off, fmt, value):
    b = bytearray(rec)
    struct.pack_into(fmt, b, off, value)
    return bytes(b)


RECORD_CASES = {
    "magic": (0, "<I", 0x12345678),
    "layer": (4, "<H", 7),
    "expert": (6, "<H", 5),
    "fmt_vq4p": (8, "<B", 8),
    "fmt_q4g": (8, "<B", 3),
    "lowrank": (12, "<H", 1),
    "codebook_over": (10, "<H", 10),
    "blocks": (16, "<I", 1),
    "gate_off": (20, "<I", 52),
    "offsets_unordered": (24, "<I", 10 ** 6),
    "corr_past_end": (32, "<I", 1 << 30),
    "corr_unordered": (32, "<I", 100),
}


@pytest.mark.parametrize("case", sorted(RECORD_CASES))
def test_record_header_refusals(tmp_path, fixture, case):
    Ls, manifest, files = fixture
    off, fmt, v = RECORD_CASES[case]
    rb = Ls[0].rec_bytes
    bank = bytearray(files["experts-L1.bin"])
    e = 3
    bank[e * rb:(e + 1) * rb] = _patch(Ls[0].records[e], off, fmt, v)
    f = dict(files)
    f["experts-L1.bin"] = bytes(bank)
    c = warp_amd.Container(make(tmp_path, manifest, f))
    assert c.read_expert(1, e - 1)[0] == 0
    assert c.read_expert(1, e)[0] == warp_amd.ERECORD
    assert c.read_expert(1, e + 1)[0] == 0
    assert c.error() == (warp_amd.ERECORD, 1, e)
    # first failure wins
    assert c.read_expert(1, 99)[0] == warp_amd.EINVAL
    assert c.error() == (warp_amd.ERECORD, 1, e)


def test_vq2r_record_accepted_by_the_reader(tmp_path, fixture):
    """record_check takes VQ2R beside VQ3R at index_bits 8."""
    Ls, manifest, files = fixture
    rb = Ls[0].rec_bytes
    bank = bytearray(files["experts-L1.bin"])
    bank[0:rb] = _patch(Ls[0].records[0], 8, "<B", 5)
    f = dict(files)
    f["experts-L1.bin"] = bytes(bank)
    assert warp_amd.Container(make(tmp_path, manifest, f)).read_expert(1, 0)[0] == 0


def test_vq4p_round_trip(tmp_path):
    """A VQ4P container (expert_quant VQ4P, index_bits 6: four stages of 64
    entries, twelve books a layer): its config, books and records read back
    as written, and a VQ3R record in it is refused (model.c:3660-3666)."""
    Ls = [Layer(H, I, E, K, seed=120 + r, cb_base=12 * r, layer=1 + r, score_func=1, n_shared=1,
                shared_fmt=FMT_Q8G, index_bits=6) for r in range(2)]
    manifest, files = build(Ls, n_layers=3, first_dense=1)
    c = warp_amd.Container(make(tmp_path, manifest, files), verify=True)
    cfg = c.config()
    assert (cfg["stages"], cfg["vec_dim"], cfg["entries"], cfg["index_bits"]) == (4, 8, 64, 6)
    assert cfg["n_books"] == 24
    books = c.codebooks()
    assert books.shape == (24, 64, 8)
    for r, Lyr in enumerate(Ls):
        n, cb, rb = c.bank(1 + r)
        assert (n, cb, rb) == (E, 12 * r, Lyr.rec_bytes)
        assert np.array_equal(books[cb:cb + 12], Lyr.books_f16[cb:cb + 12])
        for e in range(E):
            rc, rec = c.read_expert(1 + r, e)
            assert rc == 0 and rec.tobytes() == Lyr.records[e]
    bank = bytearray(files["experts-L1.bin"])
    bank[0:Ls[0].rec_bytes] = _patch(Ls[0].records[0], 8, "<B", 4)
    f = dict(files)
    f["experts-L1.bin"] = bytes(bank)
    assert warp_amd.Container(make(tmp_path, manifest, f, "c2")).read_expert(1, 0)[0] == warp_amd.ERECORD


def test_swapped_records(tmp_path, fixture):
    """A bank whose records are out of order is caught by the identity
    check, never served as another expert."""
    Ls, manifest, files = fixture
    rb = Ls[0].rec_bytes
    bank = bytearray(files["experts-L2.bin"])
    bank[0:rb], bank[rb:2 * rb] = bank[rb:2 * rb], bank[0:rb]
    f = dict(files)
    f["experts-L2.bin"] = bytes(bank)
    c = warp_amd.Container(make(tmp_path, manifest, f))
    assert c.read_expert(2, 0)[0] == warp_amd.ERECORD
    assert c.read_expert(2, 1)[0] == warp_amd.ERECORD
    assert c.read_expert(2, 2)[0] == 0


def test_checksum_on_request(tmp_path, fixture):
    """A flipped payload bit passes the header checks and fails the crc32
    only when verify is on; the 4 KiB padding is not covered."""
    Ls, manifest, files = fixture
    rb = Ls[0].rec_bytes
    e = 5
    rec = Ls[0].records[e]
    corr = struct.unpack_from("<I", rec, 32)[0]
    end = corr + 2 * (2 * I + H)                        # payload end: the last row scale
    assert struct.unpack_from("<I", rec, 36)[0] == zlib.crc32(rec[48:end])
    assert end < rb, "the fixture's records need padding"
    bank = bytearray(files["experts-L1.bin"])
    bank[e * rb + 4000] ^= 0x10                         # record e's index payload
    bank[e * rb - 1] ^= 0xFF                            # record e - 1's padding
    f = dict(files)
    f["experts-L1.bin"] = bytes(bank)
    path = make(tmp_path, manifest, f)
    assert warp_amd.Container(path).read_expert(1, e)[0] == 0
    c = warp_amd.Container(path, verify=True)
    assert c.read_expert(1, e - 1)[0] == 0
    assert c.read_expert(1, e)[0] == warp_amd.ECRC
    assert c.error() == (warp_amd.ECRC, 1, e)


def test_fuzzed_manifests_never_crash(tmp_path, fixture):
    """Byte-level mutations of a good manifest: open either refuses or the
    container reads back without fault (tools/fuzz_container.py's job)."""
    Ls, manifest, files = fixture
    path = make(tmp_path, manifest, files)
    good = json.dumps(manifest).encode()
    rng = np.random.default_rng(5)
    codes = set()
    for it in range(300):
        b = bytearray(good)
        for _ in range(int(rng.integers(1, 4))):
            i = int(rng.integers(0, len(b)))
            op = int(rng.integers(0, 3))
            if op == 0:
                b[i] = int(rng.integers(32, 127))
            elif op == 1:
                del b[i]
            else:
                b.insert(i, int(rng.choice(list(b'0123456789-e.{}[]",:'))))
        with open(os.path.join(path, "manifest.json"), "wb") as f:
            f.write(bytes(b))
        rc = opened(path)
        codes.add(rc)
        assert rc in (0, warp_amd.EFORMAT, warp_amd.EIO, warp_amd.ENOMEM), rc
        if rc == 0:
            c = warp_amd.Container(path)
            for L in range(3):
                if c.bank(L):
                    for e in range(c.bank(L)[0]):
                        c.read_expert(L, e)
            for t in manifest["trunk"]:
                try:
                    c.tensor(t["name"])
                except warp_amd.HipError:
                    pass
            c.close()
    assert 0 in codes and warp_amd.EFORMAT in codes


def test_reader_under_asan(tmp_path, fixture):
    """The reader's C sources built with AddressSanitizer and UBSan on the
    host, run over the same fuzzed manifests and a damaged bank."""
    Ls, manifest, files = fixture
    here = os.path.dirname(os.path.abspath(__file__))
    host = os.path.join(here, "..", "warp_amd", "csrc", "host")
    exe = str(tmp_path / "fuzz")
    subprocess.check_call(["gcc", "-std=gnu11", "-g", "-O1", "-fsanitize=address,undefined",
                           "-fno-sanitize-recover=all", "-I", os.path.join(here, "..", "include"),
                           "-I", host, os.path.join(here, "container_fuzz.c"), os.path.join(host, "container.c"),
                           os.path.join(host, "json.c"), os.path.join(host, "crc32.c"), "-o", exe, "-lpthread",
                           "-lm"])
    path = make(tmp_path, manifest, files)
    bank = bytearray(files["experts-L1.bin"])
    bank[Ls[0].rec_bytes + 32] ^= 0x7                   # corr offset of expert 1
    with open(os.path.join(path, "experts-L1.bin"), "wb") as f:
        f.write(bytes(bank))
    r = subprocess.run([exe, path, "400", "11"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    assert "opened" in r.stdout, r.stdout


@pytest.mark.parametrize("group_limit", [False, True])
def test_oracle_from_container(tmp_path, group_limit):
    """The oracle's layer built from the reader's output equals the one
    built from the writer's arrays, bit for bit: logits, selection,
    weights and output."""
    Ls = layers(n_group=4, topk_group=2)
    manifest, files = build(Ls, n_layers=3, first_dense=1)
    c = warp_amd.Container(make(tmp_path, manifest, files), verify=True)
    orc = Oracle()
    for r, Lw in enumerate(Ls):
        view = oracle_view(c, 1 + r, group_limit)
        if not group_limit:
            Lw.n_group = Lw.topk_group = 1
        a, b = orc.moe(view, 0), orc.moe(Lw, 0)
        for t in range(3):
            x = Lw.inputs(1, seed=40 + t)[0]
            ra, ya, ia, wa, la = a.layer(x)
            rb, yb, ib, wb, lb = b.layer(x)
            assert ra == rb == 0
            assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))


# ---- a container the reference's own tool wrote -------------------------

def ref_container(tmp_path):
    """tests/golden/ref_container.npz (tests/golden/make_ref_container.py:
    the reference's tools/make_test_container.py, seed 0) unpacked into a
    directory."""
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_container.npz"))
    d = tmp_path / "ref"
    d.mkdir()
    for name in g.files:
        (d / name).write_bytes(g[name].tobytes())
    return str(d), {name: g[name].tobytes() for name in g.files}


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def test_reference_written_container(tmp_path, orc):
    """The reader on a container written by the reference's tooling: the
    config against the manifest's JSON, every record crc-checked and equal
    to its slice of the bank file, the codebooks against the file's
    per-book layout (a 16-byte waste_codebook_hdr, then 256 x 8 f16,
    src/waste_format.h:139-150), the MoE trunk tensors against their
    manifest offsets, and the oracle's layer on what the reader returned."""
    path, raw = ref_container(tmp_path)
    man = json.loads(raw["manifest.json"])
    jc = man["config"]
    c = warp_amd.Container(path, verify=True)
    cfg = c.config()
    assert (cfg["n_layers"], cfg["hidden"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"]) == (
        jc["num_hidden_layers"], jc["hidden_size"], jc["num_experts"], jc["num_experts_per_token"],
        jc["moe_intermediate_size"])
    assert (cfg["n_shared"], cfg["first_dense"], cfg["score_func"], cfg["renorm"]) == (
        jc["num_shared_experts"], jc["first_k_dense_replace"], 0, 1)
    assert cfg["routed_scale"] == np.float32(jc["routed_scaling_factor"])
    eq = man["expert_quant"]
    assert (cfg["stages"], cfg["vec_dim"], cfg["entries"], cfg["index_block"]) == (
        eq["stages"], eq["vec_dim"], eq["entries"], eq["index_block"])
    # codebooks: book i at i * (16 + 256*8*2) + 16
    books = c.codebooks()
    cbf = raw["codebooks.bin"]
    per = 16 + 256 * 8 * 2
    assert books.shape[0] * per == len(cbf)
    for i in range(books.shape[0]):
        want = np.frombuffer(cbf[i * per + 16:(i + 1) * per], np.uint16).reshape(256, 8)
        assert np.array_equal(books[i], want), i
    # banks and records
    trunk = raw["trunk.bin"]
    tmap = {t["name"]: t for t in man["trunk"]}
    for ls, lay in man["layers"].items():
        L = int(ls)
        n, cb, rb = c.bank(L)
        assert (n, cb, rb * n) == (lay["experts"], lay["codebook_base"], lay["bytes"])
        bank = raw[lay["file"]]
        for e in range(n):
            rc, rec = c.read_expert(L, e)
            assert rc == 0 and rec.tobytes() == bank[e * rb:(e + 1) * rb], (L, e)
            buf = np.ascontiguousarray(rec, np.uint8)
            assert orc.lib.orc_record_check(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), rb, L, e,
                                            cfg["moe_inter"], cfg["hidden"], 3, books.shape[0], 1) == 0, (L, e)
        dst = np.zeros((n, rb), np.uint8)
        assert c.read_bank(L, dst) == 0 and dst.tobytes() == bank
        p = f"model.layers.{L}.block_sparse_moe."
        for name in ("gate.weight", "gate.e_score_correction_bias", "shared_experts.gate_proj.weight",
                     "shared_experts.up_proj.weight", "shared_experts.down_proj.weight"):
            ent = tmap[p + name]
            t = c.tensor(p + name)
            assert t.fmt == ent["fmt"], name
            if ent["fmt"] == 0:
                want = np.frombuffer(trunk[ent["off"]:ent["off"] + ent["bytes"]], np.float32)
                assert np.array_equal(np.asarray(t.q).reshape(-1), want), name
            else:
                rows, cols = ent["shape"]
                q = np.asarray(t.q).view(np.uint8)
                assert q.size == rows * t.rowbytes, name
                assert q.tobytes() == trunk[ent["off"]:ent["off"] + rows * t.rowbytes], name
                ng = (cols + ent["group"] - 1) // ent["group"]
                so = ent["scale_off"]
                assert np.array_equal(np.asarray(t.qs).reshape(-1),
                                      np.frombuffer(trunk[so:so + rows * ng * 2], np.uint16)), name
        # the oracle's moe_layer on the reader's view of the layer
        view = oracle_view(c, L, group_limit=False)
        x = np.random.default_rng(L).standard_normal(cfg["hidden"]).astype(np.float32)
        rc, out, idx, w, _ = orc.moe(view, 1).layer(x)
        assert rc == 0 and np.all(np.isfinite(out)) and len(set(idx.tolist())) == cfg["top_k"], L
    assert c.error() == (0, 0, 0)
    c.close()
