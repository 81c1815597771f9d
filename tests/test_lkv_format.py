"""LKV2 snapshot format on the host (no GPU): the library's reader and
writer (tqkv_lkv_check / _manifest / _rewrite) against an independent Python
writer (struct + zlib), and the reference's fault sweeps
(crates/lumen-mlx/tests/kv_disk_faults.rs) on the same sample snapshot:
every truncation and every single-byte flip is a typed error, trailing
bytes, a garbage manifest, bad magic / version and an implausible record
length are rejected and named, and a known-good file still reads after each.
"""
import os
import random
import struct
import sys
import zlib

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "lumen-rs_amd"))
import tqkv as T  # noqa: E402

import lkv_py as L  # noqa: E402


def sample():
    """kv_disk_faults.rs:25-52: two layers, an F32 [2, 4] and a BF16 [3]
    record."""
    m = L.manifest("test-fingerprint", 1_700_000_000, 42, [1, 2, 3, 4], 5, True,
                   [L.layer("Full", 0), L.layer("Linear", 1)])
    recs = [(L.DTYPES["F32"], [2, 4], b"".join(struct.pack("<f", float(i)) for i in range(8))),
            (L.DTYPES["BF16"], [3], b"".join(struct.pack("<H", 0x3F80 + i) for i in range(3)))]
    return m, recs


def corrupt_status(data):
    try:
        T.lkv_check(data)
    except T.TqkvError as e:
        return e.status, str(e)
    return T.OK, ""


def test_crc32_matches_zlib():
    rng = random.Random(3)
    assert T.crc32(b"123456789") == 0xCBF43926  # the CRC-32 check value
    assert T.crc32(b"") == 0
    for n in [1, 2, 3, 7, 64, 1000, 4097]:
        b = bytes(rng.randrange(256) for _ in range(n))
        assert T.crc32(b) == zlib.crc32(b)


def test_valid_snapshot_round_trips():
    m, recs = sample()
    data = L.write(m, recs)
    T.lkv_check(data)
    js, n_layers, n_records = T.lkv_manifest(data)
    assert (n_layers, n_records) == (2, 2)
    assert js.encode() == L.manifest_bytes(m)
    # The library's writer re-serializes the parsed manifest byte for byte as
    # serde_json does (compact, declaration order, None options skipped).
    assert T.lkv_rewrite(data) == data
    m2, r2 = L.read(T.lkv_rewrite(data))
    assert m2 == m and r2 == [(d, s, b) for d, s, b in recs]


def test_every_truncation_errors_without_panicking():
    m, recs = sample()
    data = L.write(m, recs)
    json_len = struct.unpack_from("<I", data, 8)[0]
    boundaries = [4, 8, 12, 12 + json_len, 16 + json_len, 20 + json_len]
    offsets = sorted(set(range(len(data))) | {b + d for b in boundaries for d in (-1, 0, 1)
                                               if 0 <= b + d < len(data)})
    assert len(offsets) > 100
    for off in offsets:
        status, _ = corrupt_status(data[:off])
        assert status == T.ECORRUPT, f"truncation at {off}/{len(data)} parsed as valid"
        T.lkv_check(data)  # the good input still reads


def test_every_single_byte_flip_is_rejected():
    m, recs = sample()
    data = L.write(m, recs)
    for at in range(len(data)):
        bad = bytearray(data)
        bad[at] ^= 0xFF
        status, _ = corrupt_status(bytes(bad))
        assert status == T.ECORRUPT, f"a flip at byte {at}/{len(data)} read back as valid"
    T.lkv_check(data)


def test_trailing_bytes_are_rejected():
    m, recs = sample()
    status, msg = corrupt_status(L.write(m, recs) + b"\0")
    assert status == T.ECORRUPT and "trailing" in msg


def test_garbage_manifest_errors():
    m, recs = sample()
    data = bytearray(L.write(m, recs))
    json_len = struct.unpack_from("<I", data, 8)[0]
    data[12:12 + json_len] = b"#" * json_len
    status, msg = corrupt_status(bytes(data))
    assert status == T.ECORRUPT and "manifest" in msg
    # With a CRC that matches the garbage, the JSON parse names it.
    junk = b"#" * json_len
    status, msg = corrupt_status(L.write(m, recs, raw_json=junk))
    assert status == T.ECORRUPT and "manifest" in msg


def test_bad_magic_and_version_are_named():
    m, recs = sample()
    data = L.write(m, recs)
    status, msg = corrupt_status(b"XXXX" + data[4:])
    assert status == T.ECORRUPT and "magic" in msg
    status, msg = corrupt_status(data[:4] + struct.pack("<I", 99) + data[8:])
    assert status == T.ECORRUPT and "version" in msg and "99" in msg


def test_implausible_record_length_is_rejected_not_allocated():
    m, recs = sample()
    data = L.write(m, recs)
    json_len = struct.unpack_from("<I", data, 8)[0]
    rec0 = 12 + json_len + 8
    ndim = struct.unpack_from("<I", data, rec0 + 1)[0]
    at = rec0 + 1 + 4 + ndim * 4
    for claimed in [2 ** 64 - 1, (2 ** 64 - 1) // 2, 1 << 40]:
        bad = data[:at] + struct.pack("<Q", claimed) + data[at + 8:]
        status, _ = corrupt_status(bad)
        assert status == T.ECORRUPT
    # A shape whose product overflows is refused the same way.
    big = L.write(m, [(L.DTYPES["U64"], [2 ** 31 - 1] * 8, b"")])
    status, msg = corrupt_status(big)
    assert status == T.ECORRUPT and "record" in msg


@pytest.mark.parametrize("mutate,needle", [
    (lambda d: d.pop("position"), "position"),
    (lambda d: d.pop("layers"), "layers"),
    (lambda d: d["layers"][0].pop("kind"), "kind"),
    (lambda d: d["layers"][0].update(kind="Sideways"), "variant"),
    (lambda d: d.update(position=-1), "position"),
    (lambda d: d.update(position=1.5), "position"),
    (lambda d: d.update(prefix_tokens=[2 ** 32]), "prefix_tokens"),
    (lambda d: d["layers"][0].update(group_size=2 ** 31), "group_size"),
    (lambda d: d.update(is_deep=1), "is_deep"),
])
def test_manifest_fields_are_checked(mutate, needle):
    m, recs = sample()
    mutate(m)
    status, msg = corrupt_status(L.write(m, recs))
    assert status == T.ECORRUPT and "deserialize manifest" in msg and needle in msg, msg


def test_duplicate_field_and_unknown_field():
    m, recs = sample()
    js = L.manifest_bytes(m)
    dup = js[:-1] + b',"position":7}'
    status, msg = corrupt_status(L.write(m, recs, raw_json=dup))
    assert status == T.ECORRUPT and "duplicate" in msg
    extra = js[:-1] + b',"note":{"a":[1,2,{"b":null}]}}'
    T.lkv_check(L.write(m, recs, raw_json=extra))  # serde ignores unknown fields


def test_rewrite_canonical_form_with_every_option():
    layers = [
        L.layer("SlidingQuantized", 5000, 0, [0, 1, None, 3], max_size=1024, keep=0, idx=17,
                bits=4, group_size=64),
        L.layer("FullTurboquant", 77, 3, [None, None], max_size=2 ** 64 - 1, keep=4, idx=9,
                bits=3, qjl_m=128),
        L.layer("Linear", 2, 0, [], lengths_id=1, left_padding_id=0),
    ]
    m = L.manifest("fp \"quoted\" \\ \x01\t\n é☃", 2 ** 64 - 1, 0, [], None, False, layers)
    recs = [(L.DTYPES["U8"], [0], b""), (L.DTYPES["I64"], [2, 1], struct.pack("<2q", -1, 2)),
            (L.DTYPES["Bool"], [], b""), (L.DTYPES["BF16"], [1, 2, 1, 1], b"\x80\x3f\x80\xbf")]
    data = L.write(m, recs)
    assert T.lkv_rewrite(data) == data
    js, nl, nr = T.lkv_manifest(data)
    assert (nl, nr) == (3, 4) and js.encode() == L.manifest_bytes(m)
    # Non-canonical spacing and order still parse; the rewrite canonicalizes.
    loose = b'{ "layers": [ ], "is_deep": false, "prefix_tokens": [ 9 ],\n' \
            b'  "position": 1, "created_at_unix": 2, "model_fingerprint": "\\u0041\\ud83d\\ude00" }'
    want = L.manifest("A\U0001F600", 2, 1, [9], None, False, [])
    assert L.read(T.lkv_rewrite(L.write(None, [], raw_json=loose)))[0] == want
    assert T.lkv_rewrite(L.write(None, [], raw_json=loose)) == L.write(want, [])
