"""Writes tests/golden/mlx_qwen4exp_tiny.npz: real MLX quantize and
dequantize output taken from the reference's qwen4exp_tiny fixture
(crates/lumen-mlx/tests/fixtures/qwen4exp_tiny, produced with mlx 0.32.4 by
scripts/golden/qwen4exp_tiny_fixture.py; README.md:17-19, 39-41, 70).

The safetensors files are read as data only: the 8-byte header length, the
JSON header, then raw little-endian arrays at the offsets it names. Nothing
is imported from or executed in the reference.

What the .npz holds:
  embed_w / embed_s / embed_b   language_model.model.embed_tokens as MLX
                                 quantized it: u32 [128, 8], f32 [128, 2] x 2
                                 (4-bit, group 32, f32 scales and biases)
  mtp_ids                       int32 [48] (reference/mtp_outputs.safetensors)
  mtp_embedded                  f32 [47, 64]: MLX's dequantize of the
                                 embedding rows mtp_ids[1:]
                                 (qwen4exp_tiny_fixture.py:318, 362)
  q4_w / q4_s / q4_b            4-bit group-32 groups of the quantized
                                 weights (u32 [n, 4], f32 [n], f32 [n]): every
                                 SAMPLE_STRIDE-th group of each tensor, in file
                                 order over model.safetensors then
                                 mtp.safetensors
  q8_w / q8_s / q8_b            every 8-bit group-64 group of both files
                                 (u32 [n, 16], f32 [n], f32 [n])
  q4_src / q8_src               index into `names` of each group's tensor
  names                         tensor names

Usage: python tests/golden/make_mlx_fixture.py [<reference root>]
"""
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE_DIR = "crates/lumen-mlx/tests/fixtures/qwen4exp_tiny"
SAMPLE_STRIDE = 8
DTYPES = {"F32": np.float32, "U32": np.uint32, "I32": np.int32, "I64": np.int64}


def read_safetensors(path):
    """{name: array} of a safetensors file, parsed from its bytes."""
    with open(path, "rb") as f:
        blob = f.read()
    (n,) = struct.unpack("<Q", blob[:8])
    header = json.loads(blob[8:8 + n])
    base = 8 + n
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        lo, hi = meta["data_offsets"]
        dt = np.dtype(DTYPES[meta["dtype"]]).newbyteorder("<")
        out[name] = np.frombuffer(blob[base + lo:base + hi], dtype=dt).reshape(meta["shape"])
    return out


def quant_plan(config):
    """{tensor base: (bits, group size)} from a fixture's quantization map."""
    q = config["quantization"]
    default = (q["bits"], q["group_size"])
    return default, {k: (v["bits"], v["group_size"]) for k, v in q.items() if isinstance(v, dict)}


def groups_of(tensors, default, overrides, prefix=""):
    """(name, bits, gs, words [n, W], scales [n], biases [n]) per quantized tensor."""
    for name in sorted(tensors):
        if not name.endswith(".weight") or tensors[name].dtype != np.uint32:
            continue
        base = name[:-len(".weight")]
        if base + ".scales" not in tensors:
            continue
        bits, gs = overrides.get(prefix + base, default)
        w = tensors[name]
        s = tensors[base + ".scales"]
        b = tensors[base + ".biases"]
        words = gs * bits // 32
        assert w.shape[-1] * 32 // bits == s.shape[-1] * gs, name
        yield (name, bits, gs, w.reshape(-1, words), s.reshape(-1), b.reshape(-1))


def main(ref_root):
    d = os.path.join(ref_root, FIXTURE_DIR)
    model = read_safetensors(os.path.join(d, "model.safetensors"))
    mtp = read_safetensors(os.path.join(d, "mtp.safetensors"))
    outs = read_safetensors(os.path.join(d, "reference", "mtp_outputs.safetensors"))
    with open(os.path.join(d, "config.json")) as f:
        m_default, m_over = quant_plan(json.load(f))
    with open(os.path.join(d, "mtp.json")) as f:
        mj = json.load(f)
    t_default = (4, mj["group_size"])
    t_over = {k: (v["bits"], v["group_size"]) for k, v in mj["quantization"].items()
              if k != "default"}

    names, q4, q8 = [], [], []
    for tensors, default, over in ((model, m_default, m_over), (mtp, t_default, t_over)):
        for name, bits, gs, w, s, b in groups_of(tensors, default, over):
            idx = len(names)
            names.append(name)
            if (bits, gs) == (4, 32):
                sel = slice(0, None, SAMPLE_STRIDE)
                q4.append((w[sel], s[sel], b[sel], np.full(len(s[sel]), idx, np.int32)))
            elif (bits, gs) == (8, 64):
                q8.append((w, s, b, np.full(len(s), idx, np.int32)))
            else:
                raise ValueError(f"{name}: unexpected bits {bits} group {gs}")

    def cat(parts, i):
        return np.ascontiguousarray(np.concatenate([p[i] for p in parts]))

    emb = "language_model.model.embed_tokens"
    out = os.path.join(HERE, "mlx_qwen4exp_tiny.npz")
    np.savez_compressed(
        out,
        embed_w=np.ascontiguousarray(model[emb + ".weight"]),
        embed_s=np.ascontiguousarray(model[emb + ".scales"]),
        embed_b=np.ascontiguousarray(model[emb + ".biases"]),
        mtp_ids=np.ascontiguousarray(outs["mtp_ids"].reshape(-1)),
        mtp_embedded=np.ascontiguousarray(outs["mtp_embedded"].reshape(47, 64)),
        q4_w=cat(q4, 0), q4_s=cat(q4, 1), q4_b=cat(q4, 2), q4_src=cat(q4, 3),
        q8_w=cat(q8, 0), q8_s=cat(q8, 1), q8_b=cat(q8, 2), q8_src=cat(q8, 3),
        names=np.array(names),
    )
    print(f"wrote {out}: {len(cat(q4, 1))} 4-bit gs32 groups, {len(cat(q8, 1))} 8-bit gs64 "
          f"groups, {os.path.getsize(out)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
