"""Quantize-on-append and fused decode on the GPU, through the C ABI, against
the CPU oracle: packed codes, scales and biases bit-exact; attention within
2e-2 max-abs and 1e-3 mean-abs in bf16 (|got - RN_bf16(expected)|, tests/bars.py)
of dequantize-then-attend with the exact dequantization the reference's
decode paths use, and at cosine >= 0.9999 of
attention over the mlx::dequantize'd (bf16) cache, the reference's own bar for
its fused kernel (native_quant_attention.rs:353-403)."""
import numpy as np
import pytest

import oracle_lib as O
from bars import MAX_ABS, MEAN_ABS, check_bf16
from inputs import grid_bf16, kv_bf16

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def quantize_gpu(T, x, gs, bits, dst_cap=None, dst_start=0):
    """x: bf16 [slabs, s, dim] -> device triple [slabs, cap, .] as numpy."""
    slabs, s, dim = x.shape
    cap = s if dst_cap is None else dst_cap
    dx = T.DeviceArray.of(x)
    words, groups = dim * bits // 32, dim // gs
    pk = T.DeviceArray((slabs, cap, words), np.uint32, np.full((slabs, cap, words), 0xDEADBEEF, np.uint32))
    sc = T.DeviceArray((slabs, cap, groups), np.uint16, np.full((slabs, cap, groups), 0x7777, np.uint16))
    bi = T.DeviceArray((slabs, cap, groups), np.uint16, np.full((slabs, cap, groups), 0x7777, np.uint16))
    print(f"[quantize] slabs={slabs} s={s} dim={dim} gs={gs} bits={bits} cap={cap}", flush=True)
    T.affine_quantize(dx.ptr, slabs, s, dim, gs, bits, pk.ptr, sc.ptr, bi.ptr, cap, dst_start)
    T.hip().sync()
    return pk.numpy(), sc.numpy(), bi.numpy()


@pytest.mark.parametrize("dim,gs,bits", [
    (64, 64, 4), (128, 64, 4), (128, 64, 3), (256, 64, 3), (128, 64, 8), (256, 32, 4),
    (512, 128, 8), (1024, 64, 4), (32, 32, 4), (128, 64, 2), (128, 64, 6), (128, 32, 5),
    (256, 128, 3),
])
@pytest.mark.parametrize("kind", ["normal_outliers", "golden_grid"])
def test_quantize_bit_exact(T, dim, gs, bits, kind):
    shape = (3, 37, dim)
    x = kv_bf16(shape, 100 + dim + bits, frac=0.02, mult=8.0) if kind == "normal_outliers" \
        else grid_bf16(shape, 200 + dim + bits)
    pk, sc, bi = quantize_gpu(T, x, gs, bits)
    wpk, wsc, wbi = O.affine_quantize(x, gs, bits)
    assert np.array_equal(sc, wsc)
    assert np.array_equal(bi, wbi)
    assert np.array_equal(pk, wpk)


def test_quantize_writes_only_its_rows(T):
    x = kv_bf16((4, 5, 128), 7)
    pk, sc, bi = quantize_gpu(T, x, 64, 4, dst_cap=16, dst_start=9)
    wpk, wsc, wbi = O.affine_quantize(x, 64, 4)
    assert np.array_equal(pk[:, 9:14], wpk) and np.array_equal(sc[:, 9:14], wsc)
    assert np.all(pk[:, :9] == 0xDEADBEEF) and np.all(pk[:, 14:] == 0xDEADBEEF)
    assert np.all(sc[:, :9] == 0x7777) and np.all(bi[:, 14:] == 0x7777)


def device_triple(T, slabs, cap, dim, gs, bits):
    words, groups = dim * bits // 32, dim // gs
    return (T.DeviceArray((slabs, cap, words), np.uint32,
                          np.full((slabs, cap, words), 0xDEADBEEF, np.uint32)),
            T.DeviceArray((slabs, cap, groups), np.uint16,
                          np.full((slabs, cap, groups), 0x7777, np.uint16)),
            T.DeviceArray((slabs, cap, groups), np.uint16,
                          np.full((slabs, cap, groups), 0x7777, np.uint16)))


@pytest.mark.parametrize("dim,gs,bk,bv,slabs,s", [
    (128, 64, 8, 4, 3, 37), (256, 64, 3, 3, 2, 29), (64, 32, 4, 2, 5, 1), (1024, 128, 8, 5, 2, 9),
    (32, 32, 6, 4, 7, 3), (128, 64, 4, 4, 4, 33000),  # the last loops over its grid
])
def test_quantize_kv_one_launch_matches_two(T, dim, gs, bk, bv, slabs, s):
    """tqkv_affine_quantize_kv: K and V bit-exact with the oracle (and so with
    two tqkv_affine_quantize calls), rows outside [start, start + s) untouched."""
    start, cap = 3, s + 5
    k = kv_bf16((slabs, s, dim), 300 + dim + bk, frac=0.02, mult=8.0)
    v = kv_bf16((slabs, s, dim), 400 + dim + bv, frac=0.02, mult=8.0)
    dk, dv = T.DeviceArray.of(k), T.DeviceArray.of(v)
    kt, vt = device_triple(T, slabs, cap, dim, gs, bk), device_triple(T, slabs, cap, dim, gs, bv)
    print(f"[quantize_kv] slabs={slabs} s={s} dim={dim} gs={gs} bits={bk}/{bv}", flush=True)
    T.affine_quantize_kv(dk.ptr, dv.ptr, slabs, s, dim, gs, bk, bv, tuple(a.ptr for a in kt),
                         tuple(a.ptr for a in vt), cap, start)
    T.hip().sync()
    for x, trip, bits in ((k, kt, bk), (v, vt, bv)):
        got = [a.numpy() for a in trip]
        want = O.affine_quantize(x, gs, bits)
        for g, w, fill in zip(got, want, (0xDEADBEEF, 0x7777, 0x7777)):
            assert np.array_equal(g[:, start:start + s], w)
            assert np.all(g[:, :start] == fill) and np.all(g[:, start + s:] == fill)


@pytest.mark.parametrize("dim,gs,bk,bv,slabs,s", [
    (128, 64, 4, 4, 8, 4096),   # config 0's append (K rotated, V as is)
    (128, 32, 3, 8, 3, 37), (128, 128, 8, 2, 2, 15), (256, 64, 4, 3, 2, 29),
    (256, 128, 5, 4, 1, 1), (256, 32, 6, 6, 3, 50),
])
def test_quantize_rotated(T, dim, gs, bk, bv, slabs, s):
    """tqkv_affine_quantize_rotated / _kv_rotated: the affine + rotation mode
    (gemma4_moe.rs:4154-4173) in one pass. rotate_last_axis is an f32 x f32
    matmul cast to bf16 whose summation order is MLX's (open): every rotated
    element must be within the error bound of an f32 sum in any order plus
    half a bf16 step of the f64 product (a dropped term or a transposed R is
    far outside it), over 99% equal to the f64 product's bf16 rounding, and
    the codes, scales and biases
    bit-exact with the oracle's quantizer on the kernel's own rotated rows;
    V (not rotated, as the reference leaves it) bit-exact with the oracle;
    rows outside [start, start + s) untouched."""
    start, cap = 5, s + 9
    print(f"[quantize-rot] dim={dim} gs={gs} bits={bk}/{bv} slabs={slabs} s={s}", flush=True)
    k = kv_bf16((slabs, s, dim), 500 + dim + bk, frac=0.02, mult=8.0)
    v = kv_bf16((slabs, s, dim), 600 + dim + bv, frac=0.02, mult=8.0)
    R = O.rotation(dim, 42)
    dk, dv, dR = T.DeviceArray.of(k), T.DeviceArray.of(v), T.DeviceArray.of(R)
    rot = T.DeviceArray((slabs, s, dim), np.uint16, np.zeros((slabs, s, dim), np.uint16))
    kt1 = device_triple(T, slabs, cap, dim, gs, bk)
    T.affine_quantize_rotated(dk.ptr, slabs, s, dim, gs, bk, dR.ptr, *(a.ptr for a in kt1), cap,
                              start, rot.ptr)
    kt, vt = device_triple(T, slabs, cap, dim, gs, bk), device_triple(T, slabs, cap, dim, gs, bv)
    T.affine_quantize_kv_rotated(dk.ptr, dv.ptr, slabs, s, dim, gs, bk, bv, dR.ptr,
                                 tuple(a.ptr for a in kt), tuple(a.ptr for a in vt), cap, start)
    T.hip().sync()
    y = rot.numpy()
    xf = O.bf16_to_f32(k).astype(np.float64)
    exact = xf @ R.astype(np.float64)
    got = O.bf16_to_f32(y).astype(np.float64)
    # Any f32 summation order of D products is within D * 2^-24 * sum |x_k R_kc|
    # of the exact sum; the bf16 cast adds half a bf16 step of the result.
    acc_err = dim * 2.0 ** -24 * (np.abs(xf) @ np.abs(R.astype(np.float64)))
    mag = np.maximum(np.abs(exact) + acc_err, 2.0 ** -126)
    bound = acc_err + 0.5 * 2.0 ** (np.floor(np.log2(mag)) - 7)
    ratio = np.abs(got - exact) / bound
    same = np.mean(y == O.bf16_from_f32(exact.astype(np.float32)))
    print(f"[quantize-rot] rotated: max {ratio.max():.3f} of the f32-sum + bf16-cast bound, "
          f"{100 * same:.2f}% equal to the f64 product's rounding", flush=True)
    assert ratio.max() <= 1.0 and same > 0.99
    want_k = O.affine_quantize(y, gs, bk)
    want_v = O.affine_quantize(v, gs, bv)
    for trip, want in ((kt1, want_k), (kt, want_k), (vt, want_v)):
        for a, w, fill in zip(trip, want, (0xDEADBEEF, 0x7777, 0x7777)):
            g = a.numpy()
            assert np.array_equal(g[:, start:start + s], w)
            assert np.all(g[:, :start] == fill) and np.all(g[:, start + s:] == fill)


@pytest.mark.parametrize("dim", [128, 256])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_quantize_rotated_ties_and_grid(T, dim, bits):
    """With R = I the rotated rows are the input exactly (x * 1 plus exact
    zeros), so the rotate path's quantizer (which multiplies by 1 / scale
    and takes the exact division only near a rounding boundary) is checked
    against the oracle on inputs built to land on boundaries: groups
    spanning [0, n_bins] with every other value at k + 1/2 (every code a
    tie), and the golden tests' 2^-22 grid, rich in exact ties."""
    print(f"[quantize-rot-ties] dim={dim} bits={bits}", flush=True)
    top = (1 << bits) - 1
    rows = 40
    x = np.zeros((rows, dim), np.float32)
    for g in range(dim // 64):
        x[:, 64 * g] = 0.0
        x[:, 64 * g + 1] = float(top)
        x[:, 64 * g + 2:64 * (g + 1)] = (np.arange(62) % top) + 0.5
    x[::2] *= -1.0  # the other sign of every tie on half the rows
    xb = np.concatenate([O.bf16_from_f32(x), grid_bf16((rows, dim), 70 + bits)])[None]
    eye = np.eye(dim, dtype=np.float32)
    dx, dR = T.DeviceArray.of(xb), T.DeviceArray.of(eye)
    n = xb.shape[1]
    rot = T.DeviceArray((1, n, dim), np.uint16, np.zeros((1, n, dim), np.uint16))
    t = device_triple(T, 1, n, dim, 64, bits)
    T.affine_quantize_rotated(dx.ptr, 1, n, dim, 64, bits, dR.ptr, *(a.ptr for a in t), n, 0,
                              rot.ptr)
    T.hip().sync()
    y = rot.numpy()
    # x * 1 plus zeros: the input, except that -0 sums to +0.
    assert np.array_equal(y, np.where(xb == 0x8000, 0, xb).astype(np.uint16))
    for a, w in zip(t, O.affine_quantize(y, 64, bits)):
        assert np.array_equal(a.numpy(), w)


def test_quantize_rotated_refuses_other_dims(T):
    with pytest.raises(T.TqkvError) as e:
        T.affine_quantize_rotated(0, 1, 1, 64, 64, 4, 0, 0, 0, 0)
    assert e.value.status == T.EINVAL_ARG  # null pointers come first
    R = T.DeviceArray.of(O.rotation(64, 42))
    x = T.DeviceArray((1, 1, 64), np.uint16, np.zeros((1, 1, 64), np.uint16))
    t = device_triple(T, 1, 1, 64, 64, 4)
    with pytest.raises(T.TqkvError) as e:
        T.affine_quantize_rotated(x.ptr, 1, 1, 64, 64, 4, R.ptr, *(a.ptr for a in t))
    assert e.value.status == T.EUNSUPPORTED


def test_quantize_kv_rejects_either_bad_width(T):
    for bk, bv in ((7, 4), (4, 7)):
        with pytest.raises(T.TqkvError) as e:
            T.affine_quantize_kv(0, 0, 1, 1, 128, 64, bk, bv, (0, 0, 0), (0, 0, 0))
        assert e.value.status == T.EUNSUPPORTED


def test_quantize_rejects_bad_layouts(T):
    with pytest.raises(T.TqkvError) as e:
        T.affine_quantize(0, 1, 1, 96, 64, 4, 0, 0, 0)
    assert e.value.status in (T.EUNSUPPORTED, T.EINVAL_SHAPE)
    with pytest.raises(T.TqkvError) as e:
        T.affine_quantize(0, 1, 1, 128, 64, 7, 0, 0, 0)
    assert e.value.status == T.EUNSUPPORTED
    with pytest.raises(T.TqkvError) as e:
        T.affine_quantize(0, 1, 4, 128, 64, 4, 0, 0, 0, 3, 0)  # 4 rows into 3
    assert e.value.status == T.EINVAL_SHAPE


@pytest.mark.parametrize("dim,gs,bits,rows", [
    (256, 64, 3, 80), (128, 64, 4, 77), (128, 32, 2, 9), (64, 64, 5, 33), (256, 128, 6, 21),
    (512, 64, 8, 7), (32, 32, 3, 101), (1024, 128, 5, 3), (128, 128, 6, 65)])
def test_dequantize_bit_exact(T, dim, gs, bits, rows):
    """Eight values a thread (16-byte aligned output) against the oracle's
    mlx::dequantize, at every width and 32-1024 channels."""
    x = kv_bf16((1, rows, dim), 9 + bits, frac=0.01, mult=10.0)
    wpk, wsc, wbi = O.affine_quantize(x, gs, bits)
    out = T.DeviceArray((1, rows, dim), np.uint16)
    pk, sc, bi = T.DeviceArray.of(wpk), T.DeviceArray.of(wsc), T.DeviceArray.of(wbi)
    T.affine_dequantize(pk.ptr, sc.ptr, bi.ptr, rows, dim, gs, bits, out.ptr)
    T.hip().sync()
    assert np.array_equal(out.numpy(), O.affine_dequantize(wpk, wsc, wbi, gs, bits))


def test_dequantize_unaligned_output(T):
    """An output one bf16 past a 16-byte boundary takes the one-value path:
    the same bits, nothing written outside the rows."""
    rows, dim, gs, bits = 19, 128, 64, 3
    x = kv_bf16((1, rows, dim), 31, frac=0.01, mult=10.0)
    wpk, wsc, wbi = O.affine_quantize(x, gs, bits)
    buf = T.DeviceArray.of(np.full(rows * dim + 16, 0x7777, np.uint16))
    pk, sc, bi = T.DeviceArray.of(wpk), T.DeviceArray.of(wsc), T.DeviceArray.of(wbi)
    T.affine_dequantize(pk.ptr, sc.ptr, bi.ptr, rows, dim, gs, bits, buf.ptr + 2)
    T.hip().sync()
    got = buf.numpy()
    want = O.affine_dequantize(wpk, wsc, wbi, gs, bits).reshape(-1)
    assert np.array_equal(got[1:1 + rows * dim], want)
    assert got[0] == 0x7777 and np.all(got[1 + rows * dim:] == 0x7777)


# ------------------------------------------------------------------ decode
def _cache(x, gs, bits, cap=None):
    """Quantize with the oracle and upload as a [B, Hkv, cap, .] view."""
    B, Hkv, N, D = x.shape
    cap = N if cap is None else cap
    pk, sc, bi = O.affine_quantize(x, gs, bits)
    def pad(a):
        out = np.zeros((B, Hkv, cap, a.shape[-1]), a.dtype)
        out[:, :, :N] = a
        return out
    host = (pk, sc, bi)
    dev = tuple(__import__("tqkv").DeviceArray.of(pad(a)) for a in host)
    return host, dev


def run_decode(T, q, segs_host, B, H, Hkv, D, gs, bk, bv, scale):
    """segs_host: list of (k_dev, v_dev, cap, n, shared)."""
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    segs = [T.affine_seg(tuple(a.ptr for a in k), tuple(a.ptr for a in v), cap, n, sh)
            for (k, v, cap, n, sh) in segs_host]
    T.decode_attend_affine(dq.ptr, B, H, Hkv, D, gs, bk, bv, scale, segs, out.ptr)
    T.hip().sync()
    return out.numpy()


def check_close(got_bf16, want_f32, want_mlx_f32=None, tag="decode"):
    """want_f32: oracle with the exact dequantization of the reference's
    decode paths; the kernel meets the bar in bf16 against it
    (bars.check_bf16). want_mlx_f32: oracle over the mlx::dequantize'd (bf16)
    cache, what the reference's SDPA parity test compares its fused kernel
    with: cosine >= 0.9999 (native_quant_attention.rs:395)."""
    check_bf16(got_bf16, want_f32, tag)
    if want_mlx_f32 is not None:
        got = O.bf16_to_f32(got_bf16).astype(np.float64)
        c = cosine(got, want_mlx_f32)
        print(f"[{tag}] vs_mlx_dequant max_abs={np.abs(got - want_mlx_f32).max():.3e} "
              f"cos={c:.7f}", flush=True)
        assert c >= 0.9999


def bf16_ulp(x):
    """Spacing of the bf16 grid at |x| (8 significant bits)."""
    ax = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


DECODE_CASES = [
    # (B, H, Hkv, D, N, bits_k, bits_v, gs, cap_extra)
    (1, 32, 8, 128, 8192, 4, 4, 64, 0),     # config 1 shape
    (2, 16, 8, 256, 4096, 3, 3, 64, 256),    # config 2 shape, shorter context
    (1, 16, 4, 256, 4100, 4, 4, 64, 0),      # native_quant_attention.rs:377 cases
    (1, 16, 4, 256, 4100, 8, 8, 64, 0),
    (1, 24, 4, 256, 777, 4, 4, 64, 0),
    (1, 24, 8, 128, 513, 3, 3, 64, 0),
    (1, 16, 2, 256, 20, 4, 4, 64, 5),
    (1, 16, 2, 512, 9000, 8, 8, 64, 0),
    (1, 16, 8, 256, 40000, 4, 4, 64, 0),
    (2, 32, 8, 128, 3000, 8, 4, 64, 0),      # config 4 widths (K8/V4)
    (3, 8, 8, 64, 1, 4, 4, 32, 3),           # a single key
    (1, 4, 1, 128, 777, 3, 3, 32, 0),        # all heads on one KV head
    (1, 4, 4, 128, 100, 3, 8, 128, 0),
    (1, 32, 8, 128, 3000, 6, 6, 64, 0),      # 6-bit (Gemma's kv bits 6)
    (2, 16, 8, 256, 1500, 5, 5, 64, 0),      # 5-bit: bit-anchored windows
    (1, 16, 4, 128, 999, 2, 2, 32, 0),       # 2-bit
    (1, 16, 2, 512, 2000, 6, 6, 128, 0),     # 6-bit, D = 512, G = 8
    (1, 32, 4, 128, 2000, 3, 3, 64, 0),      # 3-bit, 8 heads a KV head
    (2, 24, 4, 256, 1000, 3, 3, 64, 5),      # 3-bit, 6 heads a KV head
    (1, 64, 8, 128, 1500, 6, 6, 64, 0),      # 6-bit, 8 heads a KV head
    (3, 48, 8, 64, 700, 5, 5, 32, 0),        # 5-bit, 6 heads a KV head, D = 64
    (2, 16, 8, 256, 3000, 4, 4, 32, 0),      # group size 32 at D = 256 (16 A rows)
    (1, 32, 8, 128, 2000, 4, 4, 32, 0),      # group size 32, 4 heads a KV head
    (1, 16, 8, 128, 1500, 8, 4, 128, 0),     # group size 128
    (2, 16, 4, 256, 999, 6, 6, 128, 3),      # group size 128 at D = 256
    (2, 8, 1, 64, 600, 4, 4, 32, 0),         # group size 32 at D = 64, 8 heads
    (1, 32, 2, 512, 3000, 4, 4, 64, 0),      # Gemma 4 full attention: 16 heads a KV head, D = 512
    (2, 32, 2, 128, 1500, 4, 4, 64, 0),      # 16 heads a KV head: two launches of 8
    (1, 20, 4, 128, 700, 8, 8, 64, 0),       # 5 heads a KV head: five launches of 1
    (1, 32, 1, 256, 900, 3, 3, 64, 0),       # 32 heads on one KV head
    (2, 64, 8, 256, 900, 4, 4, 64, 0),       # 8 heads at D = 256: two MFMA launches of 4
]


@pytest.fixture(params=["auto", "dot2"])
def kernel(request, monkeypatch):
    """Runs a decode test on the default kernel choice and again with the
    dot2 kernel forced, so both kernels meet the same bar."""
    if request.param == "dot2":
        monkeypatch.setenv("TQKV_DECODE_KERNEL", "dot2")
    else:
        monkeypatch.delenv("TQKV_DECODE_KERNEL", raising=False)
    return request.param


@pytest.mark.parametrize("B,H,Hkv,D,N,bk,bv,gs,extra", DECODE_CASES)
def test_decode_matches_dequantize_then_attend(T, kernel, B, H, Hkv, D, N, bk, bv, gs, extra):
    name = T.decode_kernel_name(H, Hkv, D, gs, bk, bv)
    print(f"[decode] B={B} H={H}/{Hkv} D={D} N={N} bits={bk}/{bv} gs={gs} kernel={name}",
          flush=True)
    seed = B * 1000003 + H * 1009 + D * 17 + N + bk * 7 + bv
    q = kv_bf16((B, H, 1, D), seed)
    k = kv_bf16((B, Hkv, N, D), seed + 1, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), seed + 2, frac=0.01, mult=10.0)
    scale = 1.0 / np.sqrt(D)
    (kh, kd), (vh, vd) = _cache(k, gs, bk, N + extra), _cache(v, gs, bv, N + extra)
    got = run_decode(T, q, [(kd, vd, N + extra, N, False)], B, H, Hkv, D, gs, bk, bv, scale)
    wf, _, _ = O.attend_affine(q, kh, vh, gs, bk, bv, scale)
    wm, _, _ = O.attend_affine(q, kh, vh, gs, bk, bv, scale, dequant="bf16")
    check_close(got, wf, wm)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("H,Hkv,D,N", [
    (16, 4, 256, 4100), (24, 4, 256, 777), (16, 2, 256, 20), (16, 2, 512, 9000),
    (16, 8, 256, 40000)])
def test_decode_reference_fused_kernel_cases(T, kernel, H, Hkv, D, N, bits):
    # native_quant_attention.rs:353-403: q ~ N(0, 1/D) in bf16, K/V ~ N(0, 1)
    # quantized from a buffer 256 tokens longer and read as the first N
    # (a strided view, as the cache hands it out), scale 1.0; the fused
    # kernel must agree with SDPA over the dequantized cache at cos >= 0.9999.
    print(f"[decode-ref] H={H}/{Hkv} D={D} N={N} bits={bits}", flush=True)
    seed = 0xF5ED + 100 * N + bits
    q = kv_bf16((1, H, 1, D), seed, std=D ** -0.5)
    cap = N + 256
    kbuf, vbuf = kv_bf16((1, Hkv, cap, D), seed + 1), kv_bf16((1, Hkv, cap, D), seed + 2)
    kt, vt = O.affine_quantize(kbuf, 64, bits), O.affine_quantize(vbuf, 64, bits)
    kd = tuple(T.DeviceArray.of(a) for a in kt)
    vd = tuple(T.DeviceArray.of(a) for a in vt)
    got = run_decode(T, q, [(kd, vd, cap, N, False)], 1, H, Hkv, D, 64, bits, bits, 1.0)
    cut = lambda t: tuple(np.ascontiguousarray(a[:, :, :N]) for a in t)
    wm, _, _ = O.attend_affine(q, cut(kt), cut(vt), 64, bits, bits, 1.0, dequant="bf16")
    wf, _, _ = O.attend_affine(q, cut(kt), cut(vt), 64, bits, bits, 1.0)
    c = cosine(O.bf16_to_f32(got), wm)
    print(f"[decode-ref] cos_vs_mlx_dequant={c:.7f}", flush=True)
    assert c >= 0.9999
    check_close(got, wf)


@pytest.mark.parametrize("B,H,Hkv,D,n1,n2,shared,bk,bv", [
    (2, 16, 2, 512, 700, 333, False, 4, 4),   # a ring view: two segments of one cache
    (1, 32, 2, 512, 1500, 90, True, 8, 8),    # one sequence over a shared prefix
    (2, 8, 2, 128, 513, 200, False, 4, 8),
])
def test_decode_two_segments(T, kernel, B, H, Hkv, D, n1, n2, shared, bk, bv):
    """Two segments in one softmax on every decode path (the D = 512 tile
    kernel included): the oracle over their concatenation."""
    print(f"[decode-2seg] B={B} H={H}/{Hkv} D={D} n={n1}+{n2} shared={shared} "
          f"kernel={T.decode_kernel_name(H, Hkv, D, 64, bk, bv)}", flush=True)
    gs = 64
    q = kv_bf16((B, H, 1, D), 31 + D, std=D ** -0.5 * 4)
    b1 = 1 if shared else B
    k1, v1 = kv_bf16((b1, Hkv, n1, D), 32), kv_bf16((b1, Hkv, n1, D), 33)
    k2, v2 = kv_bf16((B, Hkv, n2, D), 34), kv_bf16((B, Hkv, n2, D), 35)
    (k1h, k1d), (v1h, v1d) = _cache(k1, gs, bk, n1 + 7), _cache(v1, gs, bv, n1 + 7)
    (k2h, k2d), (v2h, v2d) = _cache(k2, gs, bk, n2 + 3), _cache(v2, gs, bv, n2 + 3)
    got = run_decode(T, q, [(k1d, v1d, n1 + 7, n1, shared), (k2d, v2d, n2 + 3, n2, False)], B,
                     H, Hkv, D, gs, bk, bv, 1.0)
    cat = lambda a, b: np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
    kfull = tuple(cat(a, b) for a, b in zip(k1h, k2h))
    vfull = tuple(cat(a, b) for a, b in zip(v1h, v2h))
    wf, _, _ = O.attend_affine(q, kfull, vfull, gs, bk, bv, 1.0)
    wm, _, _ = O.attend_affine(q, kfull, vfull, gs, bk, bv, 1.0, dequant="bf16")
    check_close(got, wf, wm)


def test_decode_shared_prefix_plus_suffix(T, kernel):
    # sdpa_split semantics (native_attention.rs:174-208): one softmax over a
    # shared batch-1 prefix and each row's own suffix.
    B, H, Hkv, D, P, S, gs = 3, 8, 2, 128, 700, 130, 64
    q = kv_bf16((B, H, 1, D), 5)
    kp, vp = kv_bf16((1, Hkv, P, D), 6), kv_bf16((1, Hkv, P, D), 7)
    ks, vs = kv_bf16((B, Hkv, S, D), 8), kv_bf16((B, Hkv, S, D), 9)
    (kph, kpd), (vph, vpd) = _cache(kp, gs, 8), _cache(vp, gs, 4)
    (ksh, ksd), (vsh, vsd) = _cache(ks, gs, 8, S + 10), _cache(vs, gs, 4, S + 10)
    got = run_decode(T, q, [(kpd, vpd, P, P, True), (ksd, vsd, S + 10, S, False)], B, H, Hkv, D,
                     gs, 8, 4, 0.1)
    kfull = tuple(np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
                  for a, b in zip(kph, ksh))
    vfull = tuple(np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
                  for a, b in zip(vph, vsh))
    wf, _, _ = O.attend_affine(q, kfull, vfull, gs, 8, 4, 0.1)
    wm, _, _ = O.attend_affine(q, kfull, vfull, gs, 8, 4, 0.1, dequant="bf16")
    check_close(got, wf, wm)


@pytest.mark.parametrize("B,H,Hkv,D,P,S,bk,bv,gs", [
    (8, 32, 8, 128, 5000, 300, 8, 4, 64),   # config 4 widths, shorter prefix
    (2, 16, 8, 256, 1000, 0, 3, 3, 64),     # prefix only
    (4, 8, 8, 64, 777, 65, 4, 4, 32),
    (5, 12, 4, 128, 2049, 1, 4, 8, 128),    # odd batch, G = 3
    (4, 32, 2, 128, 1000, 50, 4, 4, 64),    # 16 heads a KV head (suffix in two launches)
])
def test_decode_shared_prefix_read_once(T, monkeypatch, B, H, Hkv, D, P, S, bk, bv, gs):
    # With B >= 2 sequences over a shared prefix the prefix is read once per
    # KV head for all of them (MFMA over the sequences' query rows, split
    # over the prefix) and merged with each suffix's partials; the
    # per-sequence path (TQKV_SHARED_PREFIX=0) must agree, and both meet the
    # oracle's bar.
    print(f"[decode-shared] B={B} H={H}/{Hkv} D={D} P={P} S={S} bits={bk}/{bv} gs={gs}",
          flush=True)
    seed = B * 131 + D + P + S
    q = kv_bf16((B, H, 1, D), seed, std=D ** -0.5 * 4)
    kp, vp = kv_bf16((1, Hkv, P, D), seed + 1), kv_bf16((1, Hkv, P, D), seed + 2)
    ks, vs = kv_bf16((B, Hkv, S, D), seed + 3), kv_bf16((B, Hkv, S, D), seed + 4)
    (kph, kpd), (vph, vpd) = _cache(kp, gs, bk), _cache(vp, gs, bv)
    (ksh, ksd), (vsh, vsd) = _cache(ks, gs, bk, S + 3), _cache(vs, gs, bv, S + 3)
    segs = [(kpd, vpd, P, P, True), (ksd, vsd, S + 3, S, False)]
    monkeypatch.delenv("TQKV_SHARED_PREFIX", raising=False)
    got = run_decode(T, q, segs, B, H, Hkv, D, gs, bk, bv, 1.0)
    monkeypatch.setenv("TQKV_SHARED_PREFIX", "0")
    per_seq = run_decode(T, q, segs, B, H, Hkv, D, gs, bk, bv, 1.0)
    kfull = tuple(np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
                  for a, b in zip(kph, ksh))
    vfull = tuple(np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
                  for a, b in zip(vph, vsh))
    wf, _, _ = O.attend_affine(q, kfull, vfull, gs, bk, bv, 1.0)
    wm, _, _ = O.attend_affine(q, kfull, vfull, gs, bk, bv, 1.0, dequant="bf16")
    check_close(got, wf, wm)
    check_close(per_seq, wf, wm)
    d = np.abs(O.bf16_to_f32(got) - O.bf16_to_f32(per_seq))
    print(f"[decode-shared] shared vs per-sequence max={d.max():.3e}", flush=True)


def test_decode_rejects_unreadable_layouts(T):
    q = T.DeviceArray((1, 12, 1, 128), np.uint16)
    out = T.DeviceArray((1, 12, 1, 128), np.uint16)
    seg = T.affine_seg((q.ptr,) * 3, (q.ptr,) * 3, 1, 1)
    for args in [(1, 66, 2, 128, 64, 4, 4), (1, 68, 2, 128, 64, 3, 3), (1, 12, 12, 96, 32, 4, 4),
                 (1, 12, 12, 128, 64, 7, 7), (1, 12, 12, 128, 64, 5, 4), (1, 12, 12, 128, 64, 6, 8)]:
        with pytest.raises(T.TqkvError) as e:
            T.decode_attend_affine(q.ptr, *args, 1.0, [seg], out.ptr)
        assert e.value.status == T.EUNSUPPORTED, args
    with pytest.raises(T.TqkvError) as e:
        T.decode_attend_affine(q.ptr, 1, 12, 5, 128, 64, 4, 4, 1.0, [seg], out.ptr)
    assert e.value.status == T.EINVAL_SHAPE


@pytest.mark.parametrize("B,H,Hkv,D,N,bk,bv", [(2, 16, 8, 256, 4100, 3, 3), (1, 32, 8, 128, 3333, 4, 4)])
def test_decode_single_launch_path(T, kernel, monkeypatch, B, H, Hkv, D, N, bk, bv):
    # One workgroup per (batch row, KV head), normalizing in-kernel: the path
    # the full-size benchmark takes (B * H_kv fills the GPU there).
    monkeypatch.setenv("TQKV_DECODE_SPLITS", "1")
    print(f"[decode-1split] B={B} H={H}/{Hkv} D={D} N={N} bits={bk}/{bv}", flush=True)
    q = kv_bf16((B, H, 1, D), 77)
    k = kv_bf16((B, Hkv, N, D), 78, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), 79, frac=0.01, mult=10.0)
    (kh, kd), (vh, vd) = _cache(k, 64, bk, N + 7), _cache(v, 64, bv, N + 7)
    got = run_decode(T, q, [(kd, vd, N + 7, N, False)], B, H, Hkv, D, 64, bk, bv, D ** -0.5)
    wf, _, _ = O.attend_affine(q, kh, vh, 64, bk, bv, D ** -0.5)
    check_close(got, wf)


def plant_large_values(v, k, q, seed, G, frac=0.04):
    """Scales one 64-channel group of a seeded set of tokens' values by 1e3
    to 1e6 (bf16 holds them; their quantization scales pass f16's 65,504
    once weighted), and turns half of those tokens' keys towards the first
    query head of their group so that they carry the softmax weight."""
    rng = np.random.default_rng(seed)
    vf, kf, qf = O.bf16_to_f32(v).copy(), O.bf16_to_f32(k).copy(), O.bf16_to_f32(q)
    B, Hkv, N, D = v.shape
    for b in range(B):
        for h in range(Hkv):
            toks = rng.choice(N, size=max(2, int(frac * N)), replace=False)
            for i, t in enumerate(toks):
                g = rng.integers(0, D // 64)
                vf[b, h, t, g * 64:(g + 1) * 64] *= np.float32(10.0 ** rng.integers(3, 7))
                if i % 2 == 0:
                    kf[b, h, t] = qf[b, h * G, 0] * np.float32(rng.uniform(0.5, 2.0))
    return O.bf16_from_f32(vf), O.bf16_from_f32(kf)


@pytest.mark.parametrize("splits", ["auto", "1"])
@pytest.mark.parametrize("H,Hkv,D,N,bits", [
    (16, 8, 256, 1500, 3), (32, 8, 128, 1200, 4), (16, 4, 256, 900, 8)])
def test_decode_large_value_scales(T, kernel, monkeypatch, splits, H, Hkv, D, N, bits):
    # Value groups far outside N(0,1): the f16 value weights p * scale must
    # stay finite (p reaches 2^8 under the lagging maximum), so the output
    # is within the bar of the oracle relative to its own magnitude.
    if splits == "1":
        monkeypatch.setenv("TQKV_DECODE_SPLITS", "1")
    else:
        monkeypatch.delenv("TQKV_DECODE_SPLITS", raising=False)
    B, G = 2, H // Hkv
    print(f"[decode-large-v] H={H}/{Hkv} D={D} N={N} bits={bits} splits={splits}", flush=True)
    q = kv_bf16((B, H, 1, D), 4000 + bits)
    k = kv_bf16((B, Hkv, N, D), 4001 + bits, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), 4002 + bits)
    v, k = plant_large_values(v, k, q, 4003 + bits, G)
    (kh, kd), (vh, vd) = _cache(k, 64, bits, N + 3), _cache(v, 64, bits, N + 3)
    got = run_decode(T, q, [(kd, vd, N + 3, N, False)], B, H, Hkv, D, 64, bits, bits, D ** -0.5)
    want, _, _ = O.attend_affine(q, kh, vh, 64, bits, bits, D ** -0.5)
    mag = np.maximum(np.abs(want).max(axis=-1, keepdims=True), 1.0)
    print(f"[decode-large-v] max|want|={np.abs(want).max():.3e}", flush=True)
    check_bf16(got, want, "decode-large-v relative", scale=mag)
