"""An independent Python statement of the LKV2 layout (kv_disk.rs:371-448)
for the tests: a writer that builds files the way write_lkv does (serde_json
compact manifest, field order of the Rust structs, zlib's CRC-32) and a
reader that splits a file into its manifest and records. Test
infrastructure only; the library's reader and writer are checked against it.
"""
import json
import struct
import zlib

DTYPES = {"Bool": 0, "U8": 1, "U16": 2, "U32": 3, "U64": 4, "I8": 5, "I16": 6, "I32": 7,
          "I64": 8, "F16": 9, "F32": 10, "F64": 11, "BF16": 12}
ELEM = {0: 1, 1: 1, 2: 2, 3: 4, 4: 8, 5: 1, 6: 2, 7: 4, 8: 8, 9: 2, 10: 4, 11: 8, 12: 2}


def layer(kind, offset, base_offset=0, arrays=(), **opt):
    """LayerMeta as serde writes it: None options (absent here) skipped."""
    d = {"kind": kind, "offset": offset, "base_offset": base_offset, "arrays": list(arrays)}
    for k in ("lengths_id", "left_padding_id", "max_size", "keep", "idx", "bits", "qjl_m",
              "group_size"):
        if opt.get(k) is not None:
            d[k] = opt[k]
    return d


def manifest(fingerprint, created, position, prefix, last_token, is_deep, layers):
    d = {"model_fingerprint": fingerprint, "created_at_unix": created, "position": position,
         "prefix_tokens": list(prefix)}
    if last_token is not None:
        d["last_token"] = last_token
    d["is_deep"] = is_deep
    d["layers"] = list(layers)
    return d


def manifest_bytes(m):
    return json.dumps(m, separators=(",", ":"), ensure_ascii=False).encode()


def record(dtype, shape, data):
    body = struct.pack("<B", dtype) + struct.pack("<I", len(shape))
    body += b"".join(struct.pack("<i", d) for d in shape)
    body += struct.pack("<Q", len(data)) + bytes(data)
    return body + struct.pack("<I", zlib.crc32(body))


def write(m, records, raw_json=None):
    js = manifest_bytes(m) if raw_json is None else raw_json
    out = b"LKV2" + struct.pack("<I", 2) + struct.pack("<I", len(js)) + js
    out += struct.pack("<I", zlib.crc32(js)) + struct.pack("<I", len(records))
    return out + b"".join(record(*r) for r in records)


def read(buf):
    """(manifest dict, [(dtype, shape, payload bytes)]) of a well-formed file."""
    assert buf[:4] == b"LKV2" and struct.unpack_from("<I", buf, 4)[0] == 2
    n = struct.unpack_from("<I", buf, 8)[0]
    js = buf[12:12 + n]
    assert struct.unpack_from("<I", buf, 12 + n)[0] == zlib.crc32(js)
    at = 16 + n
    count = struct.unpack_from("<I", buf, at)[0]
    at += 4
    recs = []
    for _ in range(count):
        r0 = at
        dt = buf[at]
        ndim = struct.unpack_from("<I", buf, at + 1)[0]
        shape = list(struct.unpack_from("<%di" % ndim, buf, at + 5))
        at += 5 + 4 * ndim
        ln = struct.unpack_from("<Q", buf, at)[0]
        at += 8
        data = buf[at:at + ln]
        at += ln
        assert struct.unpack_from("<I", buf, at)[0] == zlib.crc32(buf[r0:at])
        at += 4
        recs.append((dt, shape, data))
    assert at == len(buf)
    return json.loads(js), recs
