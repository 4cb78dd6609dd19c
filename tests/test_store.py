"""On-disk store formats (tq_backend/cag_store.py files) through the library's
C++ entries, on the CPU.  Pinned by independent implementations: hashlib's
SHA-256, the CRC-32C check value and a bit-serial CRC, torch.save /
torch.load(weights_only=True) for the zip-pickle files, and json.dumps(indent=2)
for the manifest layout."""
from __future__ import annotations

import hashlib
import io
import json
import struct
import zipfile

import numpy as np
import pytest
import torch

from turborag_amd.cag_store import CAGStore, StoreIO
from turborag_amd.turboquant_wrapper import TQStoreFormat


@pytest.fixture(scope="module")
def sio(tq):
    return StoreIO(tq)


# ── hashes ───────────────────────────────────────────────────────────── #

@pytest.mark.parametrize("n", [0, 1, 3, 55, 56, 63, 64, 65, 119, 120, 128, 1000])
def test_sha256_matches_hashlib(sio, n):
    data = bytes((i * 37 + 11) & 0xFF for i in range(n))
    assert sio.sha256_hex(data) == hashlib.sha256(data).hexdigest()


def test_sha256_known_answer(sio):
    # FIPS 180-2 appendix B.1
    assert sio.sha256_hex(b"abc") == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"


@pytest.mark.parametrize("doc,layer,scheme", [("doc-1", 3, "turbo_prod"), ("", 0, "fp16"),
                                              ("αβγ 文書", 35, "turbo_mse"), ("x", 123, "turbo_prod"),
                                              ("neg", -1, "turbo_prod")])
def test_store_key(sio, doc, layer, scheme):
    # cag_store.py:97-100
    want = f"{hashlib.sha256(doc.encode()).hexdigest()[:16]}_L{layer:02d}_{scheme}"
    assert sio.key(doc, layer, scheme) == want


def _crc32c_bitwise(data: bytes) -> int:
    c = 0xFFFFFFFF
    for b in data:
        c ^= b
        for _ in range(8):
            c = (c >> 1) ^ (0x82F63B78 if c & 1 else 0)
    return c ^ 0xFFFFFFFF


def test_crc32c(sio):
    assert sio.crc32c(b"123456789") == 0xE3069283  # the CRC-32C check value
    rng = np.random.default_rng(5)
    for n in (0, 1, 7, 8, 9, 63, 1000):
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert sio.crc32c(d) == _crc32c_bitwise(d)


# ── .meta (torch.save zip-pickle) ────────────────────────────────────── #

@pytest.mark.parametrize("n", [0, 1, 37, 300, 70000])
def test_meta_written_here_reads_with_torch(sio, tmp_path, n):
    slots = torch.arange(n, dtype=torch.int32).flip(0)
    p = tmp_path / "a.meta"
    sio.write_meta(p, n, slots)
    d = torch.load(p, weights_only=True)
    assert set(d) == {"num_tokens", "slots"}
    assert d["num_tokens"] == n and d["slots"].dtype == torch.int32
    assert torch.equal(d["slots"], slots)


def test_meta_format_record(sio, tmp_path):
    fmt = TQStoreFormat(1, 2, 4, 64, 16, 2304, 7, 100)
    p = tmp_path / "b.meta"
    sio.write_meta(p, 100, torch.arange(100, dtype=torch.int32), fmt)
    d = torch.load(p, weights_only=True)
    assert d["tq_format"] == 1 and d["tq_scheme"] == 2 and d["num_kv_heads"] == 4
    assert d["head_dim"] == 64 and d["block_size"] == 16 and d["page_size_bytes"] == 2304
    n, s, f = sio.read_meta(p)
    assert n == 100 and torch.equal(s, torch.arange(100, dtype=torch.int32))
    assert (f.version, f.scheme, f.num_kv_heads, f.head_dim, f.block_size, f.page_size_bytes,
            f.num_tokens) == (1, 2, 4, 64, 16, 2304, 100)


@pytest.mark.parametrize("n", [0, 5, 255, 256, 65536, 100000])
def test_meta_written_by_torch_reads_here(sio, tmp_path, n):
    # what the reference writes (cag_store.py:150): torch.save of this dict
    slots = torch.randint(-5, 1 << 30, (n,), dtype=torch.int32)
    p = tmp_path / "c.meta"
    torch.save({"num_tokens": n, "slots": slots}, p)
    got_n, got_s, fmt = sio.read_meta(p)
    assert got_n == n and fmt is None
    assert torch.equal(got_s, slots)


def test_meta_tensor_view_with_offset(sio, tmp_path):
    base = torch.arange(50, dtype=torch.int32)
    p = tmp_path / "v.meta"
    torch.save({"num_tokens": 20, "slots": base[10:30]}, p)
    n, s, _ = sio.read_meta(p)
    assert n == 20 and torch.equal(s, base[10:30])


def _zip_with_pickle(path, pkl: bytes):
    with zipfile.ZipFile(path, "w", compression=zipfile.ZIP_STORED) as z:
        z.writestr("x/data.pkl", pkl)
        z.writestr("x/version", "3\n")


def test_meta_reader_rejects_code(sio, tmp_path):
    # a pickle that would call os.system under pickle.load: refused, never run
    evil = b"\x80\x02cos\nsystem\nX\x04\x00\x00\x00trueq\x00\x85R."
    p = tmp_path / "evil.meta"
    _zip_with_pickle(p, evil)
    with pytest.raises(RuntimeError, match="not allowed"):
        sio.read_meta(p)


@pytest.mark.parametrize("bad", [b"", b"not a zip at all", b"PK\x03\x04" + b"\0" * 40])
def test_meta_reader_rejects_garbage(sio, tmp_path, bad):
    p = tmp_path / "bad.meta"
    p.write_bytes(bad)
    with pytest.raises(RuntimeError):
        sio.read_meta(p)


def test_meta_reader_rejects_truncated_pickle(sio, tmp_path):
    full = io.BytesIO()
    torch.save({"num_tokens": 3, "slots": torch.arange(3, dtype=torch.int32)}, full)
    z = zipfile.ZipFile(io.BytesIO(full.getvalue()))
    pkl = z.read([n for n in z.namelist() if n.endswith("data.pkl")][0])
    p = tmp_path / "t.meta"
    _zip_with_pickle(p, pkl[:len(pkl) // 2])
    with pytest.raises(RuntimeError):
        sio.read_meta(p)


def test_meta_missing_file(sio, tmp_path):
    with pytest.raises(RuntimeError, match="cannot open"):
        sio.read_meta(tmp_path / "nope.meta")


# ── crafted archives: offsets and sizes from the file near 2^64 ──────── #

def _records_of_valid_meta(n=7):
    buf = io.BytesIO()
    torch.save({"num_tokens": n, "slots": torch.arange(n, dtype=torch.int32)}, buf)
    z = zipfile.ZipFile(io.BytesIO(buf.getvalue()))
    return [(name, z.read(name)) for name in z.namelist()]


def _hand_zip(records, patch=None):
    """A stored zip written field by field (APPNOTE 4.3.7, 4.3.12, 4.3.16).
    patch(name) may return {"lho": int, "usize": int, "csize": int,
    "zip64": [u64, ...]}: 32-bit central-directory fields to write instead of
    the true ones, and the values of a zip64 extra field (id 1)."""
    import binascii
    body, cd = b"", b""
    for name, data in records:
        nm = name.encode()
        crc = binascii.crc32(data)
        lho = len(body)
        body += struct.pack("<IHHHHHIIIHH", 0x04034B50, 20, 0, 0, 0, 0x21, crc, len(data),
                            len(data), len(nm), 0) + nm + data
        p = (patch(name) if patch else None) or {}
        extra = b""
        if "zip64" in p:
            vals = p["zip64"]
            extra = struct.pack("<HH", 1, 8 * len(vals)) + b"".join(struct.pack("<Q", v) for v in vals)
        cd += struct.pack("<IHHHHHHIIIHHHHHII", 0x02014B50, 20, 20, 0, 0, 0, 0x21, crc,
                          p.get("csize", len(data)), p.get("usize", len(data)), len(nm), len(extra),
                          0, 0, 0, 0, p.get("lho", lho)) + nm + extra
    eocd = struct.pack("<IHHHHIIH", 0x06054B50, 0, 0, len(records), len(records), len(cd),
                       len(body), 0)
    return body + cd + eocd


def test_hand_zip_helper_makes_a_readable_meta(sio, tmp_path):
    p = tmp_path / "ok.meta"
    p.write_bytes(_hand_zip(_records_of_valid_meta(7)))
    n, s, _ = sio.read_meta(p)
    assert n == 7 and torch.equal(s, torch.arange(7, dtype=torch.int32))


@pytest.mark.parametrize("lho64", [0xFFFFFFFFFFFFFFFE, 0xFFFFFFFFFFFFFFFF, 1 << 63, 0x100000000])
def test_meta_zip64_local_header_offset_past_the_file(sio, tmp_path, lho64):
    # the data.pkl record's local-header offset comes from a zip64 extra
    # field: rejected as beyond the file, not read before the buffer
    recs = _records_of_valid_meta()
    patch = lambda name: ({"lho": 0xFFFFFFFF, "zip64": [lho64]}
                          if name.endswith("data.pkl") else None)
    p = tmp_path / "lho.meta"
    p.write_bytes(_hand_zip(recs, patch))
    with pytest.raises(RuntimeError, match="beyond the file"):
        sio.read_meta(p)


@pytest.mark.parametrize("size64", [0xFFFFFFFFFFFFFF00, 0xFFFFFFFFFFFFFFFF, 1 << 40])
def test_meta_zip64_record_size_past_the_file(sio, tmp_path, size64):
    recs = _records_of_valid_meta()
    patch = lambda name: ({"usize": 0xFFFFFFFF, "csize": 0xFFFFFFFF, "zip64": [size64, size64]}
                          if name.endswith("data.pkl") else None)
    p = tmp_path / "size.meta"
    p.write_bytes(_hand_zip(recs, patch))
    with pytest.raises(RuntimeError, match="beyond the file"):
        sio.read_meta(p)


def test_meta_short_zip64_extra_field(sio, tmp_path):
    # the field claims the offset is in zip64 but carries no value for it
    recs = _records_of_valid_meta()
    patch = lambda name: {"lho": 0xFFFFFFFF, "zip64": []} if name.endswith("data.pkl") else None
    p = tmp_path / "short.meta"
    p.write_bytes(_hand_zip(recs, patch))
    with pytest.raises(RuntimeError, match="short zip64"):
        sio.read_meta(p)


@pytest.mark.parametrize("n", [0xFFFFFFFFFFFFFFF0, 0xFFFFFFFFFFFFFFFF, 1 << 63])
def test_pickle_binunicode8_huge_length(sio, tmp_path, n):
    # BINUNICODE8 (0x8d) with a length near 2^64: "truncated", and the
    # position never wraps back into the pickle
    pkl = b"\x80\x04}\x8d" + struct.pack("<Q", n) + b"num_tokens" + b"K\x05s."
    p = tmp_path / "u8.meta"
    _zip_with_pickle(p, pkl)
    with pytest.raises(RuntimeError, match="truncated"):
        sio.read_meta(p)


def _meta_pickle(shape, stride, offset=0, numel=4):
    """{"num_tokens": 1, "slots": tensor} with the tensor's shape, stride and
    storage offset as given (protocol 2, as torch.save emits it)."""
    def ints(vals):
        out = b"("
        for v in vals:
            out += b"\x8a\x08" + struct.pack("<q", v)
        return out + b"t"
    return (b"\x80\x02}(X\x0a\x00\x00\x00num_tokensK\x01X\x05\x00\x00\x00slots"
            b"ctorch._utils\n_rebuild_tensor_v2\n(("
            b"X\x07\x00\x00\x00storagectorch\nIntStorage\nX\x01\x00\x00\x000X\x03\x00\x00\x00cpu"
            + b"\x8a\x08" + struct.pack("<q", numel) + b"tQ"
            + b"\x8a\x08" + struct.pack("<q", offset) + ints(shape) + ints(stride)
            + b"\x89ccollections\nOrderedDict\n)RtRu.")


def _meta_with_tensor(path, shape, stride, offset=0, numel=4):
    with zipfile.ZipFile(path, "w", compression=zipfile.ZIP_STORED) as z:
        z.writestr("x/data.pkl", _meta_pickle(shape, stride, offset, numel))
        z.writestr("x/data/0", np.arange(numel, dtype=np.int32).tobytes())


def test_meta_tensor_pickle_helper_reads(sio, tmp_path):
    p = tmp_path / "t.meta"
    _meta_with_tensor(p, [3], [1], offset=1)
    n, s, _ = sio.read_meta(p)
    assert n == 1 and s.tolist() == [1, 2, 3]


@pytest.mark.parametrize("shape,stride,offset,msg", [
    ([1 << 62, 4], [4, 1], 0, "exceeds its storage"),         # element count overflows int64
    ([1 << 32, 1 << 32], [1 << 32, 1], 0, "exceeds its storage"),
    ([4], [1], 1 << 62, "exceeds its storage"),               # offset + n would wrap
    ([4], [1], -1, "exceeds its storage"),
    ([-4], [1], 0, "negative dimension"),
    ([2, 2], [2], 0, "ranks differ"),                          # stride shorter than shape
])
def test_meta_tensor_geometry_from_the_file_is_checked(sio, tmp_path, shape, stride, offset, msg):
    p = tmp_path / "g.meta"
    _meta_with_tensor(p, shape, stride, offset)
    with pytest.raises(RuntimeError, match=msg):
        sio.read_meta(p)


# ── fp16 scheme .bin ─────────────────────────────────────────────────── #

def test_fp16_written_here_reads_with_torch(sio, tmp_path):
    kv = torch.randn(2 * 9 * 2 * 16).half()
    p = tmp_path / "f.bin"
    sio.write_fp16(p, 9, kv, [9, 2, 16])
    d = torch.load(p, weights_only=True)
    assert d["num_tokens"] == 9 and d["shape"] == [9, 2, 16]
    assert torch.equal(d["kv"], kv)


def test_fp16_written_by_torch_reads_here(sio, tmp_path):
    kv = torch.randn(2 * 33 * 4 * 8).half()
    p = tmp_path / "g.bin"
    torch.save({"num_tokens": 33, "kv": kv, "shape": [33, 4, 8]}, p)  # cag_store.py:130
    n, got, shape = sio.read_fp16(p)
    assert n == 33 and shape == [33, 4, 8]
    assert torch.equal(got, kv)


# ── .bin pages + footer ──────────────────────────────────────────────── #

def _fmt(N=40, pages=3, page=4288):
    return TQStoreFormat(1, 1, 2, 128, 16, page, pages, N)


def test_pool_footer_and_read(sio, tmp_path):
    rng = np.random.default_rng(7)
    pool = torch.from_numpy(rng.integers(0, 256, 3 * 4288, dtype=np.uint8))
    p = tmp_path / "p.bin"
    sio.write_pool(p, pool, _fmt())
    size, fmt = sio.pool_info(p)
    assert size == pool.numel() + 64
    assert (fmt.version, fmt.scheme, fmt.num_kv_heads, fmt.head_dim, fmt.block_size,
            fmt.page_size_bytes, fmt.num_pages, fmt.num_tokens) == (1, 1, 2, 128, 16, 4288, 3, 40)
    raw = p.read_bytes()
    assert raw[:pool.numel()] == pool.numpy().tobytes()  # the reference's raw[:pool_bytes]
    magic, ver = struct.unpack_from("<8sI", raw, pool.numel())
    assert magic == b"TQPAGES\0" and ver == 1
    crc = struct.unpack_from("<I", raw, pool.numel() + 56)[0]
    assert crc == _crc32c_bitwise(pool.numpy().tobytes())
    dst = torch.zeros(pool.numel(), dtype=torch.uint8)
    sio.read_pools([p], [dst], pool.numel(), verify=True)
    assert torch.equal(dst, pool)


def test_pool_without_footer_is_read(sio, tmp_path):
    # a .bin as the reference writes it: the raw pool only (cag_store.py:147-149)
    pool = torch.arange(3 * 4288, dtype=torch.int64).remainder(251).to(torch.uint8)
    p = tmp_path / "legacy.bin"
    p.write_bytes(pool.numpy().tobytes())
    size, fmt = sio.pool_info(p)
    assert size == pool.numel() and fmt is None
    dst = torch.zeros_like(pool)
    sio.read_pools([p], [dst], pool.numel(), verify=True)
    assert torch.equal(dst, pool)


def test_pool_checksum_catches_corruption(sio, tmp_path):
    pool = torch.full((4288,), 7, dtype=torch.uint8)
    p = tmp_path / "c.bin"
    sio.write_pool(p, pool, _fmt(N=16, pages=1))
    raw = bytearray(p.read_bytes())
    raw[100] ^= 0x10
    p.write_bytes(bytes(raw))
    dst = torch.zeros_like(pool)
    sio.read_pools([p], [dst], pool.numel(), verify=False)  # unverified read succeeds
    with pytest.raises(RuntimeError, match="checksum"):
        sio.read_pools([p], [dst], pool.numel(), verify=True)


def test_read_pools_many_files_and_short_file(sio, tmp_path):
    pools = [torch.full((1000,), i, dtype=torch.uint8) for i in range(12)]
    paths = []
    for i, pl in enumerate(pools):
        paths.append(tmp_path / f"{i}.bin")
        sio.write_pool(paths[-1], pl, _fmt(N=1, pages=1, page=1000))
    dsts = [torch.zeros(1000, dtype=torch.uint8) for _ in pools]
    sio.read_pools(paths, dsts, 1000, threads=5, verify=True)
    assert all(torch.equal(a, b) for a, b in zip(dsts, pools))
    short = tmp_path / "short.bin"
    short.write_bytes(b"\0" * 10)
    with pytest.raises(RuntimeError, match="shorter"):
        sio.read_pools([short], [dsts[0]], 1000)
    with pytest.raises(ValueError):
        sio.read_pools([short], [torch.zeros(10, dtype=torch.uint8)], 1000)


# ── manifest ─────────────────────────────────────────────────────────── #

def _ref_entry(doc, layer, scheme, n, stored_at):
    """The entry cag_store.py:51-67 records."""
    h = hashlib.sha256(doc.encode()).hexdigest()
    return h, {"key": f"{h[:16]}_L{layer:02d}_{scheme}", "num_tokens": n, "stored_at": stored_at}


def test_manifest_update_layout_matches_json_dumps(sio, tmp_path):
    docs = [("doc A", 0, "turbo_prod", 100), ("doc A", 1, "turbo_prod", 100),
            ("ünïcode \"q\" \\ \n", 2, "turbo_mse", 7), ("doc A", 0, "fp16", 100)]
    for d, l, s, n in docs:
        sio.manifest_update(tmp_path, d, l, s, n)
    text = (tmp_path / "manifest.json").read_text()
    m = json.loads(text)
    # rebuild what the reference's json.dumps(manifest, indent=2) gives for the
    # same entries (stored_at taken from the file)
    want = {"v": 1, "entries": {}}
    for d, l, s, n in docs:
        stored = m["entries"][d]["layers"][f"{l}::{s}"]["stored_at"]
        assert isinstance(stored, float)
        h, e = _ref_entry(d, l, s, n, stored)
        ent = want["entries"].setdefault(d, {"sha256": h, "layers": {}})
        ent["layers"][f"{l}::{s}"] = e
    assert text == json.dumps(want, indent=2)


def test_manifest_update_preserves_reference_written_file(sio, tmp_path):
    h, e = _ref_entry("other doc", 4, "turbo_prod", 55, 1733000000.123456)
    existing = {"v": 1, "entries": {"other doc": {"sha256": h, "layers": {"4::turbo_prod": e}}},
                "extra": [1, 2.5, None, True, "s"]}
    (tmp_path / "manifest.json").write_text(json.dumps(existing, indent=2))
    sio.manifest_update(tmp_path, "other doc", 5, "turbo_prod", 55)
    m = json.loads((tmp_path / "manifest.json").read_text())
    assert m["extra"] == existing["extra"]
    assert m["entries"]["other doc"]["layers"]["4::turbo_prod"] == e
    assert m["entries"]["other doc"]["layers"]["5::turbo_prod"]["num_tokens"] == 55
    assert list(m["entries"]["other doc"]["layers"]) == ["4::turbo_prod", "5::turbo_prod"]


def test_manifest_verify(sio, tmp_path):
    sio.manifest_verify(tmp_path, "absent", 0, "turbo_prod")  # no manifest: passes
    sio.manifest_update(tmp_path, "d", 0, "turbo_prod", 10)
    sio.manifest_verify(tmp_path, "d", 0, "turbo_prod")
    sio.manifest_verify(tmp_path, "d", 9, "turbo_prod")  # no layer entry: passes
    m = json.loads((tmp_path / "manifest.json").read_text())
    m["entries"]["d"]["layers"]["0::turbo_prod"]["key"] = "wrong"
    (tmp_path / "manifest.json").write_text(json.dumps(m, indent=2))
    with pytest.raises(RuntimeError, match="Manifest key mismatch"):
        sio.manifest_verify(tmp_path, "d", 0, "turbo_prod")
    m["entries"]["d"]["sha256"] = "0" * 64
    (tmp_path / "manifest.json").write_text(json.dumps(m, indent=2))
    with pytest.raises(RuntimeError, match="Manifest integrity error"):
        sio.manifest_verify(tmp_path, "d", 0, "turbo_prod")


def test_manifest_corrupt_file_starts_fresh(sio, tmp_path):
    (tmp_path / "manifest.json").write_text("{not json")
    sio.manifest_verify(tmp_path, "d", 0, "turbo_prod")
    sio.manifest_update(tmp_path, "d", 0, "turbo_prod", 3)
    m = json.loads((tmp_path / "manifest.json").read_text())
    assert m["v"] == 1 and list(m["entries"]) == ["d"]


# ── CAGStore host-side pieces ────────────────────────────────────────── #

def test_cag_store_paths(tq, tmp_path):
    st = CAGStore(tmp_path, tq=tq)
    k = st._key("doc", 7, "turbo_mse")
    assert k == f"{hashlib.sha256(b'doc').hexdigest()[:16]}_L07_turbo_mse"
    assert st._pool_path("doc", 7, "turbo_mse").name == k + ".bin"
    assert st._meta_path("doc", 7, "turbo_mse").name == k + ".meta"
    assert not st.exists("doc", 7, "turbo_mse")
    assert st.vram_bytes("turbo_prod", 32, (2, 128)) == 2 * 4288


def test_cag_store_manifest_and_hash_helpers(tq, tmp_path):
    """The reference's private helpers (cag_store.py:32-48): the manifest
    read falls back to an empty v1 manifest for a missing or corrupt file,
    and the document hash is the SHA-256 of its UTF-8 bytes."""
    st = CAGStore(tmp_path, tq=tq)
    assert st._load_manifest() == {"v": 1, "entries": {}}
    (tmp_path / "manifest.json").write_text("{not json")
    assert st._load_manifest() == {"v": 1, "entries": {}}
    st.io.manifest_update(tmp_path, "d", 0, "turbo_prod", 12)
    assert list(st._load_manifest()["entries"]) == ["d"]
    for doc in ("doc", "", "dökümän"):
        assert st._doc_hash(doc) == hashlib.sha256(doc.encode()).hexdigest()


def test_compute_mse_matches_its_definition(tq):
    """TurboQuantWrapper.compute_mse (turboquant_wrapper.py:422): mean squared
    difference in fp32, checked on values whose squares are exact."""
    a = torch.tensor([[1.0, -2.0], [0.5, 3.0]], dtype=torch.float16)
    b = torch.tensor([[0.0, -1.0], [0.5, 1.0]], dtype=torch.float16)
    assert tq.compute_mse(a, b) == (1.0 + 1.0 + 0.0 + 4.0) / 4
    assert tq.compute_mse(a, a) == 0.0


def test_load_rejects_mismatched_footer(tq, tmp_path):
    """A .bin whose footer disagrees with the requested geometry is refused
    before anything reaches the GPU."""
    st = CAGStore(tmp_path, tq=tq)
    N = 32
    pool = torch.zeros(2 * 4288, dtype=torch.uint8)
    st.io.write_pool(st._pool_path("d", 0, "turbo_prod"), pool,
                     TQStoreFormat(1, 1, 2, 128, 16, 4288, 2, N))
    st.io.write_meta(st._meta_path("d", 0, "turbo_prod"), N, torch.arange(N, dtype=torch.int32))
    with pytest.raises(ValueError, match="stored format"):
        st.load_document("d", 0, "turbo_prod", (4, 128))
