"""The C++ host library on the CPU: hashes, the ChaCha8 word source, the WAL
format, and that both libraries export every function their headers declare.
(Session tests need the GPU and live in test_gpu_session.py.)"""
import ctypes
import hashlib
import os
import re
import struct
import zlib

import numpy as np
import pytest

import oracle_py as O
from defer_amd import gpu as G
from defer_amd import host as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str, prefix: str):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text)))


@pytest.mark.parametrize("header,prefix,path", [
    ("defer_gpu.h", "defer_gpu_", G.LIB_PATH),
    ("defer_host.h", "defer_host_", H.LIB_PATH),
])
def test_library_exports_every_declared_symbol(header, prefix, path):
    names = _declared(header, prefix)
    assert len(names) > 5
    if prefix == "defer_host_":
        G.lib()  # dependency
    lib = ctypes.CDLL(path)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_static_archive_defines_every_declared_symbol():
    """libdefer_gpu.a, the form a Rust build.rs links (static=defer_gpu),
    defines every defer_gpu_ function of include/defer_gpu.h."""
    import subprocess

    arc = os.path.join(ROOT, "defer_amd", "libdefer_gpu.a")
    out = subprocess.run(["nm", "--defined-only", "-g", arc], capture_output=True, text=True,
                         check=True).stdout
    defined = set(line.split()[-1] for line in out.splitlines() if " T " in line)
    missing = [n for n in _declared("defer_gpu.h", "defer_gpu_") if n not in defined]
    assert not missing, missing


# ------------------------------------------------------------------ hashes

def test_crc32_check_value():  # crc32.rs:34
    assert H.crc32(b"123456789") == 0xCBF43926


def test_sha256_fips_vectors():  # sha256.rs:141-158
    assert H.sha256(b"abc").hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert H.sha256(b"").hex() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    assert H.sha256(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hex() == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"


def test_hashes_match_zlib_and_hashlib_at_block_edges():
    rng = np.random.default_rng(3)
    for n in (0, 1, 55, 56, 57, 63, 64, 65, 119, 120, 128, 1000, 4099):
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert H.crc32(d) == zlib.crc32(d)
        assert H.sha256(d) == hashlib.sha256(d).digest()


# --------------------------------------------------------------- randomness

def test_host_chacha8_keystream_kat():
    want = bytes.fromhex(
        "3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"
        "984ce172b9216f419f445367456d5619314a42a3da86b001387bfdb80e0cfe42")
    assert H.chacha8_words(bytes(32), 0, 16).tobytes() == want


def test_host_words_agree_with_oracle_at_any_offset():
    seed = H.seed_from_u64(42)
    assert seed == O.seed_from_u64(42)
    for start in (0, 5, 16, 31, 1000):
        w = H.chacha8_words(seed, start, 40)
        assert [int(x) for x in w] == [O.chacha8_word(seed, start + i) for i in range(40)]


def test_words_per_sample():  # sampler.rs:15-21
    assert H.words_per_sample(0.0) == 0
    assert H.words_per_sample(0.7) == 1


# -------------------------------------------------------------------- WAL

SIG, SEED = bytes([1] * 32), bytes([2] * 32)


def test_wal_write_read_torn_resume(tmp_path):  # wal.rs:272-301
    p = str(tmp_path / "x.wal")
    w = H.Wal.create(p, SIG, SEED, 0.5, 3, 0, [10, 11, 12])
    for i, t in enumerate([5, 6, 7]):
        w.append(t, i + 1)
    w.close()
    with open(p, "ab") as f:
        f.write(bytes([1, 2, 3, 4, 5]))
    log = H.Wal.read(p)
    assert log["torn_tail"]
    assert log["history"] == [10, 11, 12, 5, 6, 7]
    assert log["rng_word_pos"] == 3
    assert log["prompt_len"] == 3 and log["temperature"] == 0.5
    w = H.Wal.resume(p, durable=True)
    assert w.next_step == 6
    w.append(8, 4)
    w.close()
    log = H.Wal.read(p)
    assert not log["torn_tail"] and log["history"][-1] == 8


def test_wal_byte_layout(tmp_path):  # wal.rs:8-31
    p = str(tmp_path / "y.wal")
    prefix = [7, 8, 9, 10]
    w = H.Wal.create(p, SIG, SEED, 0.7, 2, 0, prefix)
    w.append(99, 1)
    w.close()
    b = open(p, "rb").read()
    hdr = 104 + 4 * len(prefix)
    assert len(b) == hdr + 4 + 29
    assert b[:8] == b"DEFERWAL" and struct.unpack_from("<I", b, 8)[0] == 1
    assert b[12:44] == SIG and b[44:76] == SEED
    assert struct.unpack_from("<f", b, 76)[0] == np.float32(0.7)
    assert struct.unpack_from("<I", b, 80)[0] == 2
    assert b[84:100] == bytes(16)
    assert struct.unpack_from("<I", b, 100)[0] == len(prefix)
    assert list(struct.unpack_from("<4I", b, 104)) == prefix
    assert struct.unpack_from("<I", b, hdr)[0] == zlib.crc32(b[:hdr])
    rec = b[hdr + 4:]
    assert rec[0] == 1 and struct.unpack_from("<II", rec, 1) == (4, 99)
    assert int.from_bytes(rec[9:25], "little") == 1
    assert struct.unpack_from("<I", rec, 25)[0] == zlib.crc32(rec[:25])


def test_wal_rejects_bad_header_and_inconsistent_records(tmp_path):
    p = str(tmp_path / "z.wal")
    w = H.Wal.create(p, SIG, SEED, 0.7, 1, 0, [1])
    w.append(3, 1)
    w.append(4, 5)  # rng position must advance by one word per sample
    w.close()
    with pytest.raises(H.DeferHostError, match="inconsistent"):
        H.Wal.read(p)
    b = bytearray(open(p, "rb").read())
    b[20] ^= 0xFF
    open(p, "wb").write(bytes(b))
    with pytest.raises(H.DeferHostError, match="checksum"):
        H.Wal.read(p)
    open(p, "wb").write(b"not a wal at all, not at all, not at all" * 4)
    with pytest.raises(H.DeferHostError, match="not a defer WAL"):
        H.Wal.read(p)


def test_wal_greedy_records_keep_rng_position(tmp_path):
    p = str(tmp_path / "g.wal")
    w = H.Wal.create(p, SIG, SEED, 0.0, 2, 0, [1, 2])
    for t in (3, 4, 5):
        w.append(t, 0)
    w.close()
    log = H.Wal.read(p)
    assert log["history"] == [1, 2, 3, 4, 5] and log["rng_word_pos"] == 0


# ------------------------------------------------------------- checkpoints

def test_checkpoint_roundtrip_and_corruption(tmp_path):  # checkpoint.rs:142-156
    p = str(tmp_path / "c.ckpt")
    H.Checkpoint.save(p, bytes([7] * 32), bytes([9] * 32), 0.7, 2, 2, [1, 2, 3, 40000])
    c = H.Checkpoint.load(p)
    assert c == {"model_signature": bytes([7] * 32), "base_seed": bytes([9] * 32),
                 "temperature": float(np.float32(0.7)), "prompt_len": 2, "rng_word_pos": 2,
                 "history": [1, 2, 3, 40000]}
    b = bytearray(open(p, "rb").read())
    b[50] ^= 1
    open(p, "wb").write(bytes(b))
    with pytest.raises(H.DeferHostError, match="checksum mismatch"):
        H.Checkpoint.load(p)


def test_checkpoint_byte_layout(tmp_path):  # checkpoint.rs:4-16, 44-57
    p = str(tmp_path / "s.ckpt")
    hist = [5, 6, 7, 8, 9]
    H.Checkpoint.save(p, SIG, SEED, 0.8, 3, 2, hist)
    b = open(p, "rb").read()
    assert len(b) == 112 + 4 * len(hist)
    assert b[:8] == b"DEFERCKP" and struct.unpack_from("<I", b, 8)[0] == 1
    assert b[12:44] == SIG and b[44:76] == SEED
    assert struct.unpack_from("<f", b, 76)[0] == np.float32(0.8)
    assert struct.unpack_from("<I", b, 80)[0] == 3
    assert int.from_bytes(b[84:100], "little") == 2
    assert struct.unpack_from("<Q", b, 100)[0] == len(hist)
    assert list(struct.unpack_from("<5I", b, 108)) == hist
    assert struct.unpack_from("<I", b, len(b) - 4)[0] == zlib.crc32(b[:-4])
    assert not os.path.exists(str(tmp_path / "s.ckpt.tmp"))  # written, synced, renamed


def test_checkpoint_rejects_malformed_files(tmp_path):  # checkpoint.rs:59-84
    p = str(tmp_path / "m.ckpt")
    H.Checkpoint.save(p, SIG, SEED, 0.5, 1, 1, [4, 5])
    good = open(p, "rb").read()

    def with_crc(body):
        return body + struct.pack("<I", zlib.crc32(body))

    cases = [
        (b"NOTACKPT" + good[8:], "not a defer checkpoint"),
        (with_crc(good[:8] + struct.pack("<I", 2) + good[12:-4]), "unsupported checkpoint version"),
        (with_crc(good[:100] + struct.pack("<Q", 3) + good[108:-4]), "length mismatch"),
        (with_crc(good[:80] + struct.pack("<I", 3) + good[84:-4]), "prompt_len exceeds history"),
        (good[:60], "not a defer checkpoint"),
    ]
    for data, msg in cases:
        open(p, "wb").write(data)
        with pytest.raises(H.DeferHostError, match=msg):
            H.Checkpoint.load(p)


# ------------------------------------------------------------- model files

def _st_file(path, entries, metadata=None):
    """A safetensors file from (name, dtype, shape, raw bytes), in order."""
    import json
    hdr, off = {}, 0
    if metadata:
        hdr["__metadata__"] = metadata
    for name, dt, shape, raw in entries:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    blob = struct.pack("<Q", len(h)) + h + b"".join(e[3] for e in entries)
    open(path, "wb").write(blob)
    return blob


def test_safetensors_half_conversions(tmp_path):  # safetensors.rs:305-313
    p = str(tmp_path / "h.safetensors")
    f16 = struct.pack("<5H", 0x3C00, 0xC000, 0x7BFF, 0x0001, 0x7C00)
    bf16 = struct.pack("<2H", 0x3F80, 0xC2F7)
    f64 = struct.pack("<2d", 0.1, -3.5)
    _st_file(p, [("a", "F16", (5,), f16), ("b", "BF16", (2,), bf16), ("c", "F64", (2,), f64)])
    r = H.read_safetensors(p)
    a = r["tensors"]["a"]
    assert a[0] == 1.0 and a[1] == -2.0 and a[2] == 65504.0 and a[3] == np.float32(5.9604645e-8)
    assert np.isinf(a[4])
    assert r["tensors"]["b"][0] == 1.0 and r["tensors"]["b"][1] == np.float32(-123.5)
    assert list(r["tensors"]["c"]) == [np.float32(0.1), -3.5]
    # every f16 value against numpy's exact widening
    allh = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    _st_file(p, [("h", "F16", (65536,), allh.tobytes())])
    got = H.read_safetensors(p)["tensors"]["h"]
    want = allh.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_safetensors_order_metadata_signature(tmp_path):  # safetensors.rs:142-237
    import safetensors.numpy as stn
    p = str(tmp_path / "m.safetensors")
    rng = np.random.default_rng(0)
    t = {"z.weight": rng.standard_normal((3, 4), dtype=np.float32),
         "a.weight": rng.standard_normal((5,), dtype=np.float32),
         "m.weight": rng.standard_normal((2, 2, 2), dtype=np.float32).astype(np.float16)}
    stn.save_file(t, p, metadata={"defer.config": '{"hidden_size": 4}'})
    r = H.read_safetensors(p)
    assert r["signature"] == hashlib.sha256(open(p, "rb").read()).digest()
    assert r["defer.config"] == '{"hidden_size": 4}'
    for k, v in t.items():
        assert np.array_equal(r["tensors"][k], v.astype(np.float32))
    assert sorted(r["names"]) == sorted(t)


def test_safetensors_rejects_malformed(tmp_path):
    p = str(tmp_path / "bad.safetensors")
    raw = np.zeros(4, np.float32).tobytes()
    cases = [
        ([("a", "F32", (5,), raw)], "size mismatch for tensor a"),
        ([("a", "I8", (4,), raw[:4])], "unsupported safetensors dtype I8"),
    ]
    for entries, msg in cases:
        _st_file(p, entries)
        with pytest.raises(H.DeferHostError, match=msg):
            H.read_safetensors(p)
    open(p, "wb").write(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(H.DeferHostError, match="invalid safetensors header length"):
        H.read_safetensors(p)
    blob = _st_file(p, [("a", "F32", (4,), raw)])
    open(p, "wb").write(blob[:-3])  # data shorter than the offsets claim
    with pytest.raises(H.DeferHostError, match="out of range tensor a"):
        H.read_safetensors(p)
