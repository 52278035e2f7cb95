"""CPU tests of the GGUF reader (hyq_gguf_*, the C ABI's Gguf::open /
parse, src/gguf.rs:50-210): the reference's own tests (src/gguf.rs:312-398)
restated, SHA-256 against the FIPS 180-4 examples and Python's hashlib, and
each validation rule on a file that breaks only that rule."""
import hashlib
import math
import struct

import numpy as np
import pytest

from gguf_writer import (ARR, BOOL, F32, F64, I32, STR, U32, U64, build, string)


def tiny() -> bytes:
    """src/gguf.rs:320-335: one F32 tensor [2] = (1, -2), no metadata."""
    return build([], [("weight", [2], 0, struct.pack("<2f", 1.0, -2.0))])


def gg(hyq, b: bytes, profile: str = "auto"):
    return hyq.Gguf(data=b, profile=profile)


def test_reads_little_endian_tensor(hyq):
    g = gg(hyq, tiny())
    t = g.tensors()
    assert list(t) == ["weight"] and t["weight"]["dims"] == [2] and t["weight"]["dtype"] == 0
    assert g.tensor_bytes("weight").view(np.float32).tolist() == [1.0, -2.0]
    assert g.profile == "standard"


def test_every_truncation_is_an_error(hyq):
    b = tiny()
    for n in range(len(b)):
        with pytest.raises(ValueError):
            gg(hyq, b[:n])


def test_excessive_header_counts_fail_before_allocation(hyq):
    b = bytearray(tiny())
    b[8:16] = struct.pack("<Q", 2**64 - 1)
    with pytest.raises(ValueError, match="count exceeds"):
        gg(hyq, bytes(b))
    b = bytearray(tiny())
    b[16:24] = struct.pack("<Q", 2**40)  # metadata count
    with pytest.raises(ValueError, match="count exceeds"):
        gg(hyq, bytes(b))


@pytest.mark.parametrize("msg,digest", [
    (b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
    (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
    (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
    (b"a" * 1000000, "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"),
])
def test_sha256_fips_examples(hyq, msg, digest):
    assert hyq.sha256(msg) == digest


def test_sha256_matches_hashlib_at_every_padding_boundary(hyq):
    rng = np.random.default_rng(0)
    for n in list(range(0, 130)) + [1000, 4095, 4096, 65537]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert hyq.sha256(data) == hashlib.sha256(data).hexdigest(), n


# ---- Tencent legacy profiles (src/gguf.rs:111-153) ----

Q2C_ROW = bytes(range(130))  # one Q2_0C block = one 512-wide row
STQ_ROW = bytes(range(42))   # one STQ1_0 block = one 256-wide row
Q6K_ROW = bytes(210)


def tencent(arch="hunyuan-dense", file_type=39, ids=(40, 14, 0)):
    meta = []
    if arch is not None:
        meta.append(("general.architecture", STR, arch))
    if file_type is not None:
        meta.append(("general.file_type", U32, file_type))
    rows = {40: ([512, 1], Q2C_ROW), 42: ([256, 1], STQ_ROW), 14: ([256, 1], Q6K_ROW),
            0: ([4], bytes(16)), 12: ([256, 1], bytes(144))}
    tensors = [(f"t{i}", rows[i][0], i, rows[i][1]) for i in ids]
    return build(meta, tensors)


def test_legacy_ids_in_an_unknown_file_are_ambiguous(hyq):
    b = tencent()
    with pytest.raises(ValueError, match="ambiguous") as e:
        gg(hyq, b, "auto")
    assert hashlib.sha256(b).hexdigest() in str(e.value)


def test_legacy_ids_have_no_format_under_the_standard_profile(hyq):
    with pytest.raises(ValueError, match="unsupported GGUF tensor type 40"):
        gg(hyq, tencent(), "standard")
    with pytest.raises(ValueError, match="unsupported GGUF tensor type 42"):
        gg(hyq, tencent(file_type=41, ids=(42,)), "standard")


def test_tencent_profiles_resolve_their_ids(hyq):
    g = gg(hyq, tencent(), "tencent-q2-0c")
    assert g.profile == "tencent-q2-0c"
    t = g.tensors()
    assert t["t40"]["dtype"] == 40 and t["t40"]["byte_len"] == 130 and t["t14"]["dtype"] == 14
    g = gg(hyq, tencent(file_type=41, ids=(42, 0)), "tencent-stq1")
    assert g.profile == "tencent-stq1" and g.tensors()["t42"]["dtype"] == 42


@pytest.mark.parametrize("kw,match", [
    (dict(arch=None), "require hunyuan-dense"), (dict(arch="hy_v3"), "require hunyuan-dense"),
    (dict(file_type=None), "file_type"), (dict(file_type=41), "file_type"),
    (dict(ids=(14, 0)), "no tensors for selected"), (dict(ids=(40, 12)), "mixed types"),
])
def test_tencent_profile_rules(hyq, kw, match):
    with pytest.raises(ValueError, match=match):
        gg(hyq, tencent(**kw), "tencent-q2-0c")


def test_auto_without_legacy_ids_is_standard(hyq):
    assert gg(hyq, tencent(ids=(14, 0, 12)), "auto").profile == "standard"


# ---- header, metadata and tensor rules (src/gguf.rs:60-210, 290-388) ----

def F32_T(name="w", n=4, offset=None):
    t = (name, [n], 0, bytes(4 * n))
    return t if offset is None else t + (offset,)


@pytest.mark.parametrize("mutate,match", [
    (lambda b: b"GGUG" + b[4:], "not a GGUF file"),
    (lambda b: b[:4] + struct.pack("<I", 2) + b[8:], "v3"),
])
def test_magic_and_version(hyq, mutate, match):
    with pytest.raises(ValueError, match=match):
        gg(hyq, mutate(build([], [F32_T()])))


@pytest.mark.parametrize("meta,ok", [
    ([("general.alignment", U32, 64)], True), ([("general.alignment", U64, 1)], True),
    ([("general.alignment", U32, 48)], False), ([("general.alignment", U32, 0)], False),
    ([("general.alignment", U32, 131072)], False), ([("general.alignment", F32, 32.0)], False),
    ([("split.count", U32, 1)], True), ([("split.count", U32, 2)], False),
])
def test_alignment_and_split_rules(hyq, meta, ok):
    align = meta[0][2] if meta[0][0] == "general.alignment" and ok else 32
    b = build(meta, [F32_T("a"), F32_T("b")], alignment=int(align))
    if ok:
        g = gg(hyq, b)
        assert all(t["offset"] % align == 0 for t in g.tensors().values())
    else:
        with pytest.raises(ValueError):
            gg(hyq, b)


@pytest.mark.parametrize("tensors,match", [
    ([F32_T("a"), F32_T("a")], "duplicate tensor"),
    ([("a", [], 0, b"")], "invalid rank"),
    ([("a", [1, 1, 1, 1, 1], 0, bytes(4))], "invalid rank"),
    ([("a", [4, 0], 0, b"")], "zero dimension"),
    ([F32_T("a", offset=16)], "unaligned"),
    ([("a", [33, 1], 8, bytes(68))], "partial quantization block"),
    ([F32_T("a", offset=0), F32_T("b", offset=0)], "overlapping"),
    ([("a", [4], 7, bytes(16))], "unsupported GGUF tensor type 7"),
])
def test_tensor_rules(hyq, tensors, match):
    with pytest.raises(ValueError, match=match):
        gg(hyq, build([], tensors))


def test_truncated_tensor_data(hyq):
    b = build([], [F32_T("a", 8)])
    with pytest.raises(ValueError, match="truncated tensor"):
        gg(hyq, b[:-4])


def raw_meta(key: bytes, kind: int, payload: bytes) -> bytes:
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)
    return head + string(key) + struct.pack("<I", kind) + payload


@pytest.mark.parametrize("blob,match", [
    (raw_meta(b"k", F32, struct.pack("<f", math.nan)), "non-finite"),
    (raw_meta(b"k", F64, struct.pack("<d", math.inf)), "non-finite"),
    (raw_meta(b"k", BOOL, b"\x02"), "boolean"),
    (raw_meta(b"k", STR, string(b"\xff\xfe")), "UTF-8"),
    (raw_meta(b"k", STR, string(b"\xc0\x80")), "UTF-8"),          # overlong NUL
    (raw_meta(b"k", STR, string(b"\xed\xa0\x80")), "UTF-8"),      # surrogate
    (raw_meta(b"\xe2\x82", U32, struct.pack("<I", 1)), "UTF-8"),  # key cut mid-character
    (raw_meta(b"k", ARR, struct.pack("<IQ", ARR, 0)), "element type"),
    (raw_meta(b"k", ARR, struct.pack("<IQ", 13, 0)), "element type"),
    (raw_meta(b"k", ARR, struct.pack("<IQ", U32, 10**9)), "count exceeds"),
    (raw_meta(b"k", 13, b""), "metadata type"),
])
def test_metadata_rules(hyq, blob, match):
    with pytest.raises(ValueError, match=match):
        gg(hyq, blob)


def test_duplicate_metadata_key(hyq):
    with pytest.raises(ValueError, match="duplicate metadata key"):
        gg(hyq, build([("k", U32, 1), ("k", U32, 2)], []))


def test_metadata_accessors(hyq):
    g = gg(hyq, build([("u", U32, 7), ("neg", I32, -3), ("pos", I32, 5), ("f", F32, 0.5),
                       ("b", BOOL, True), ("s", STR, "héllo"),
                       ("a", ARR, (STR, ["x", "yz", ""])), ("big", U64, 2**63)], []))
    assert g.u64("u") == 7 and g.u64("pos") == 5 and g.u64("big") == 2**63
    with pytest.raises(ValueError):
        g.u64("neg")  # as_u64 of a negative integer
    with pytest.raises(ValueError):
        g.u64("f")
    assert g.f64("u") == 7.0 and g.f64("neg") == -3.0 and g.f64("f") == 0.5
    assert g.boolean("b") is True and g.string("s") == "héllo" and g.array_len("a") == 3
    with pytest.raises(ValueError):
        g.string("u")
    with pytest.raises(ValueError):
        g.u64("missing")


def test_tensors_are_listed_in_name_order(hyq):
    g = gg(hyq, build([], [F32_T("zeta"), F32_T("alpha"), F32_T("mid")]))
    assert list(g.tensors()) == ["alpha", "mid", "zeta"]


def test_mutated_files_open_or_fail_cleanly(hyq):
    """Seeded byte mutations of a file with metadata of every kind and two
    tensors (single bytes set, runs overwritten, cut or extended): each one
    either opens, and then every accessor answers or raises ValueError, or is
    rejected with ValueError. The reader takes untrusted files; under a
    host-AddressSanitizer build of the library this also checks that no
    mutation reads outside the file."""
    base = build([("general.architecture", STR, "hunyuan"), ("u", U32, 7), ("i", I32, -3),
                  ("f", F32, 0.5), ("d", F64, 2.5), ("b", BOOL, True), ("big", U64, 2**40),
                  ("a", ARR, (STR, ["x", "yz", ""])), ("n", ARR, (U32, [1, 2, 3]))],
                 [("w0", [4, 2], 0, struct.pack("<8f", *range(8))),
                  ("w1", [3], 0, struct.pack("<3f", 1.0, 2.0, 3.0))])
    gg(hyq, base).close()
    rng = np.random.default_rng(2024)
    opened = 0
    for _ in range(1500):
        b = bytearray(base)
        kind = rng.integers(4)
        if kind == 0:
            b[rng.integers(len(b))] = int(rng.integers(256))
        elif kind == 1:
            at = int(rng.integers(len(b)))
            run = rng.integers(0, 256, int(rng.integers(1, 9)), dtype=np.uint8).tobytes()
            b[at:at + len(run)] = run
        elif kind == 2:
            del b[int(rng.integers(len(b))):]
        else:
            b += rng.integers(0, 256, int(rng.integers(1, 64)), dtype=np.uint8).tobytes()
        try:
            g = gg(hyq, bytes(b))
        except ValueError:
            continue
        opened += 1
        for name in g.tensors():
            g.tensor_bytes(name)
        for key, get in (("u", g.u64), ("i", g.f64), ("d", g.f64), ("b", g.boolean),
                         ("general.architecture", g.string), ("a", g.array_len),
                         ("n", g.array_len), ("big", g.u64)):
            try:
                get(key)
            except ValueError:
                pass
        g.close()
    assert opened > 0  # some mutations leave a valid file (tensor data, string bytes)
