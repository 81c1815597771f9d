"""The oracle's MLX affine arithmetic against real MLX output recorded in the
reference's qwen4exp_tiny fixture (mlx 0.32.4; README.md:17-19, 39-41, 70),
extracted into tests/golden/mlx_qwen4exp_tiny.npz by
tests/golden/make_mlx_fixture.py.

- Dequantize: reference/mtp_outputs.safetensors' mtp_embedded is MLX's
  dequantize of the embedding table's rows mtp_ids[1:]
  (qwen4exp_tiny_fixture.py:318, 362; QuantizedEmbedding). It must equal the
  oracle's single fused rounding bit for bit, and the product-then-sum
  reading must not (it misses about half the elements), so the test tells
  the two apart.
- Quantize: model.safetensors and mtp.safetensors hold MLX's quantize of
  random f32 weights at 4-bit group 32 and 8-bit group 64 with f32 scales
  and biases. The original weights are not recorded, so what pins the
  quantizer is that every group whose codes span the full range is a fixed
  point: dequantized and quantized again by the oracle it gives back the
  same codes, scale and bias. Every group also carries the edge snapping's
  marks (a code 0, and bias / scale an integer).
"""
import os

import numpy as np
import pytest

import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "mlx_qwen4exp_tiny.npz")
REF_FIXTURE_DIR = "/root/reference/crates/lumen-mlx/tests/fixtures/qwen4exp_tiny"


@pytest.fixture(scope="module")
def fx():
    with np.load(FIXTURE, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def codes_of(words, bits, n):
    """Codes of each row of an LSB-first u32 stream (offload/lowbit.rs:220-240)."""
    rows = words.shape[0]
    out = np.empty((rows, n), np.uint32)
    for i in range(n):
        bit = i * bits
        w, off = bit // 32, bit % 32
        v = words[:, w].astype(np.uint64) >> np.uint64(off)
        if off + bits > 32:
            v |= words[:, w + 1].astype(np.uint64) << np.uint64(32 - off)
        out[:, i] = (v & np.uint64((1 << bits) - 1)).astype(np.uint32)
    return out


def test_dequantize_is_one_fused_rounding(fx):
    ids = fx["mtp_ids"][1:]
    w, s, b = fx["embed_w"][ids], fx["embed_s"][ids], fx["embed_b"][ids]
    got = O.affine_dequantize_f32(w, s, b, 32, 4)
    want = fx["mtp_embedded"]
    assert got.shape == want.shape == (47, 64)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # The other reading: the product rounded to f32, then the sum.
    c = codes_of(w, 4, 64).astype(np.float32)
    two = np.repeat(s, 32, axis=1) * c + np.repeat(b, 32, axis=1)
    match = np.mean(two.view(np.uint32) == want.view(np.uint32))
    print(f"product-then-sum matches {match:.1%} of mtp_embedded")
    assert match < 0.9


def test_dequantize_bf16_is_single_rounding_of_the_f32_result():
    """For bf16 scales the oracle's primary reading is bf16(f32(s c + b)):
    exactly the fused form (the product is exact in f32), rounded once."""
    rng = np.random.default_rng(5)
    for bits in (2, 3, 4, 5, 6, 8):
        x = O.bf16_from_f32(rng.standard_normal((64, 128)).astype(np.float32) * 3)
        p, s, b = O.affine_quantize(x, 64, bits)
        one = O.affine_dequantize(p, s, b, 64, bits)
        f32 = O.affine_dequantize_f32(p, O.bf16_to_f32(s), O.bf16_to_f32(b), 64, bits)
        assert np.array_equal(one, O.bf16_from_f32(f32))


def fixed_point(words, s, b, bits, gs):
    """(full-range mask, codes equal, scales equal, biases equal) after
    dequantize (fused, f32) then the oracle's f32 quantize, per group."""
    codes = codes_of(words, bits, gs)
    full = (codes.min(axis=1) == 0) & (codes.max(axis=1) == (1 << bits) - 1)
    x = O.affine_dequantize_f32(words, s[:, None], b[:, None], gs, bits)
    p2, s2, b2 = O.affine_quantize_f32(x, gs, bits)
    return (full, np.all(p2 == words, axis=1), s2[:, 0].view(np.uint32) == s.view(np.uint32),
            b2[:, 0].view(np.uint32) == b.view(np.uint32))


def snapping_marks(words, s, b, bits, gs):
    codes = codes_of(words, bits, gs)
    ratio = (b.astype(np.float64) / s.astype(np.float64))
    return codes.min(axis=1) == 0, np.abs(ratio - np.round(ratio)) <= 1e-5 * np.maximum(1, np.abs(ratio))


@pytest.mark.parametrize("tag,bits,gs", [("q4", 4, 32), ("q8", 8, 64)])
def test_quantize_fixed_point_on_mlx_output(fx, tag, bits, gs):
    w, s, b = fx[tag + "_w"], fx[tag + "_s"], fx[tag + "_b"]
    full, ceq, seq, beq = fixed_point(w, s, b, bits, gs)
    n = int(full.sum())
    print(f"{tag}: {n} of {len(s)} groups span the full range; codes {int(ceq[full].sum())}, "
          f"scales {int(seq[full].sum())}, biases {int(beq[full].sum())} identical")
    assert n >= (50 if bits == 8 else 5000)
    assert ceq[full].all() and seq[full].all() and beq[full].all()
    zero, integral = snapping_marks(w, s, b, bits, gs)
    assert zero.all() and integral.all()


def test_fixture_pins_the_scale_sign_rule(fx):
    """The check has teeth: MLX's scale is negative unless |w_min| > |w_max|
    (the bias is then the group's maximum), and the fixture holds many groups
    of each sign, so a quantizer with a positive scale and bias = min, as a
    plain min-max quantizer has, would store reversed codes for a large share
    of them and fail the fixed point. (The fixture has no all-negative or
    all-positive group, so the w_max start and the rounding of halves are
    pinned by the golden digests, not here.)"""
    for tag, bits, gs in (("q4", 4, 32), ("q8", 8, 64)):
        w, s, b = fx[tag + "_w"], fx[tag + "_s"], fx[tag + "_b"]
        neg = s < 0
        assert 0.2 < neg.mean() < 0.8, tag
        x = O.affine_dequantize_f32(w, s[:, None], b[:, None], gs, bits)
        # Negative scale: the bias is the group's largest value, else its smallest.
        assert np.array_equal(b[neg], x[neg].max(axis=1))
        assert np.array_equal(b[~neg], x[~neg].min(axis=1))


@pytest.mark.skipif(not os.path.isdir(REF_FIXTURE_DIR), reason="reference checkout absent")
def test_quantize_fixed_point_every_group_of_the_reference_files():
    """Every group of both files, not only the committed sample (runs where
    the reference checkout is present; the files are parsed as data)."""
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_mlx_fixture as M
    import json
    totals = {}
    with open(os.path.join(REF_FIXTURE_DIR, "config.json")) as f:
        m_default, m_over = M.quant_plan(json.load(f))
    with open(os.path.join(REF_FIXTURE_DIR, "mtp.json")) as f:
        mj = json.load(f)
    t_over = {k: (v["bits"], v["group_size"]) for k, v in mj["quantization"].items()
              if k != "default"}
    for fname, default, over in (("model.safetensors", m_default, m_over),
                                 ("mtp.safetensors", (4, mj["group_size"]), t_over)):
        tensors = M.read_safetensors(os.path.join(REF_FIXTURE_DIR, fname))
        for name, bits, gs, w, s, b in M.groups_of(tensors, default, over):
            full, ceq, seq, beq = fixed_point(w, s, b, bits, gs)
            zero, integral = snapping_marks(w, s, b, bits, gs)
            assert ceq[full].all() and seq[full].all() and beq[full].all(), name
            assert zero.all() and integral.all(), name
            t = totals.setdefault((bits, gs), [0, 0])
            t[0] += int(full.sum())
            t[1] += len(s)
    print({f"{k[0]}-bit gs{k[1]}": f"{v[0]} full-range of {v[1]}" for k, v in totals.items()})
    assert totals[(4, 32)][0] > 60000 and totals[(8, 64)][0] > 100
