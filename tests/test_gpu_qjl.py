"""QJL stage 2 on the GPU through the C ABI (survey row a6/a9), against the
oracle:

- the CPU path's estimator: tqkv_qjl_project_query and
  tqkv_tq_scores_two_stage are bit-exact with estimate_inner_products
  (compressor.rs:122-159, qjl.rs:76-118) on keys compressed by compress_one;
- the GPU path: tqkv_qjl_encode_stage2 and tqkv_qjl_apply_correction are
  bit-exact with the oracle's restatement of turboquant.rs:592-691, and
  meet the reference's own tests of that path: the packed-sign K_eff equals
  the bf16 +-1 path (MSE < 1e-6, turboquant.rs:1107-1178), and the
  variance / bias trade-off of qjl_m_sweep_traces_variance_threshold
  (turboquant.rs:1044-1105: MSE ratio ~ D pi / (2 m) at m < 256 within 30%,
  QJL beating stage 1 at m = 1024);
- attention over a codebook cache with QJL signs (tqkv_decode_attend_codebook_qjl)
  within 2e-2 / 1e-3 of the oracle's two-stage attention.
"""
import numpy as np
import pytest

import oracle_lib as O
from bars import check_bf16
from inputs import kv_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


@pytest.mark.parametrize("dim,bits,m", [(64, 3, 64), (128, 4, 100), (256, 4, 512), (128, 2, 32)])
def test_two_stage_scores_bit_exact(T, dim, bits, m):
    print(f"[qjl-scores] dim={dim} bits={bits} m={m}", flush=True)
    n = 77
    R, phi = T.rotation_matrix(dim, 42), T.qjl_matrix(dim, m, 43)
    _, cent = T.lloyd_max(bits)
    x = np.random.default_rng(dim + m).standard_normal((n, dim)).astype(np.float32)
    x[n // 3] = 0.0  # r_norm < 1e-10: no correction
    comp = O.Compressor(dim, bits, m, R, phi)
    s1, s2, rn, sc = comp.compress(x)
    codes = np.stack([O.unpack_codes(s1[i], dim, bits) for i in range(n)]).astype(np.uint8)
    W = (m + 31) // 32
    words = s2.view(np.uint32).reshape(n, -1)[:, :W]
    q = np.random.default_rng(7).standard_normal(dim).astype(np.float32)
    dR, dphi, dq = T.DeviceArray.of(R), T.DeviceArray.of(phi), T.DeviceArray.of(q)
    rq, pq = T.DeviceArray((dim,), np.float32), T.DeviceArray((m,), np.float32)
    T.tq_rotate_query(dR.ptr, dq.ptr, dim, rq.ptr)
    T.qjl_project_query(dphi.ptr, m, dim, dq.ptr, pq.ptr)
    dcodes, dsig = T.DeviceArray.of(codes), T.DeviceArray.of(sc)
    dsg, drn = T.DeviceArray.of(np.ascontiguousarray(words)), T.DeviceArray.of(rn)
    dcent = T.DeviceArray.of(cent.astype(np.float32))
    out = T.DeviceArray((n,), np.float32)
    T.tq_scores_two_stage(rq.ptr, pq.ptr, dcodes.ptr, dsig.ptr, dcent.ptr, dsg.ptr, drn.ptr, dim, m,
                          n, out.ptr)
    T.hip().sync()
    want = comp.scores(q, (s1, s2, rn, sc), two_stage=True)
    assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32))
    stage1 = comp.scores(q, (s1, s2, rn, sc), two_stage=False)
    assert out.numpy()[n // 3] == stage1[n // 3]  # the zero vector keeps stage 1 only


def stage1_bf16(x_bf16, bits):
    """The GPU path's stage 1 on the host (lloyd_max_quantize_stage1_fused,
    turboquant.rs:405-439; lloyd_max_dequantize_scaled, :428-439):
    sigma = sqrt(mean x^2), codes of bf16(x / sigma) against the f32
    boundaries, K_dq = bf16(centroid * sigma)."""
    x = O.bf16_to_f32(x_bf16).astype(np.float32)
    sigma = np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)).astype(np.float32)
    y = O.bf16_to_f32(O.bf16_from_f32(x / np.maximum(sigma, np.float32(1e-30))))
    import tqkv
    b, c = tqkv.lloyd_max(bits)
    inner = b[1:-1].astype(np.float32)
    codes = np.searchsorted(inner, y, side="right")
    return O.bf16_from_f32(c.astype(np.float32)[codes] * sigma)


@pytest.mark.parametrize("D,m", [(128, 64), (256, 128), (64, 100)])
def test_gpu_path_encode_and_correction_bit_exact(T, D, m):
    print(f"[qjl-gpu-path] D={D} m={m}", flush=True)
    rows = 45
    k = kv_bf16((rows, D), D + m)
    kdq = stage1_bf16(k, 4)
    phi = T.qjl_matrix(D, m, 43)
    dk, ddq, dphi = T.DeviceArray.of(k), T.DeviceArray.of(kdq), T.DeviceArray.of(phi)
    W = (m + 31) // 32
    sg, rn = T.DeviceArray((rows, W), np.uint32), T.DeviceArray((rows,), np.float32)
    T.qjl_encode_stage2(dk.ptr, ddq.ptr, dphi.ptr, rows, D, m, sg.ptr, rn.ptr)
    keff = T.DeviceArray((rows, D), np.uint16)
    T.qjl_apply_correction(ddq.ptr, sg.ptr, rn.ptr, dphi.ptr, rows, D, m, keff.ptr)
    T.hip().sync()
    wsg, wrn = O.qjl_encode_stage2(k, kdq, phi, m)
    assert np.array_equal(sg.numpy(), wsg)
    assert np.array_equal(rn.numpy().view(np.uint32), wrn.view(np.uint32))
    weff = O.qjl_apply_correction(kdq, wsg, wrn, phi, m)
    assert np.array_equal(keff.numpy(), weff)
    # The reference's packed-vs-bf16 test: the same K_eff from +-1 signs
    # through an f32 matmul.
    bits = ((sg.numpy()[:, np.arange(m) // 32] >> (np.arange(m) % 32)) & 1).astype(np.float32)
    signs_pm1 = 2.0 * bits - 1.0
    scale = np.float32(np.sqrt(np.float32(np.pi / 2)) / np.sqrt(np.float32(m)))
    corr = O.bf16_from_f32((signs_pm1 @ phi.astype(np.float32)) * (rn.numpy()[:, None] * scale))
    k_eff_bf = O.bf16_from_f32(O.bf16_to_f32(kdq) + O.bf16_to_f32(corr))
    mse = np.mean((O.bf16_to_f32(keff.numpy()) - O.bf16_to_f32(k_eff_bf)) ** 2)
    assert mse < 1e-6, mse


def test_gpu_path_variance_threshold(T):
    """turboquant.rs:1044-1105 on the device path: K [1, 4, 64, 256] N(0,1),
    4-bit stage 1; the K_eff / K_dq MSE ratio follows D pi / (2 m) below
    m = 256 (within 30%) and drops below 1 at m = 1024."""
    D, rows = 256, 4 * 64
    k = kv_bf16((rows, D), 0x1234)
    kdq = stage1_bf16(k, 4)
    kt = O.bf16_to_f32(k).astype(np.float64)
    mse_dq = np.mean((O.bf16_to_f32(kdq) - kt) ** 2)
    ratios = {}
    for m in (64, 128, 1024):
        phi = T.qjl_matrix(D, m, 43)
        dk, ddq, dphi = T.DeviceArray.of(k), T.DeviceArray.of(kdq), T.DeviceArray.of(phi)
        W = (m + 31) // 32
        sg, rn = T.DeviceArray((rows, W), np.uint32), T.DeviceArray((rows,), np.float32)
        keff = T.DeviceArray((rows, D), np.uint16)
        T.qjl_encode_stage2(dk.ptr, ddq.ptr, dphi.ptr, rows, D, m, sg.ptr, rn.ptr)
        T.qjl_apply_correction(ddq.ptr, sg.ptr, rn.ptr, dphi.ptr, rows, D, m, keff.ptr)
        T.hip().sync()
        ratios[m] = np.mean((O.bf16_to_f32(keff.numpy()) - kt) ** 2) / mse_dq
    print(f"[qjl-sweep] ratios={ratios}", flush=True)
    for m in (64, 128):
        assert abs(ratios[m] / (D * np.pi / 2 / m) - 1.0) < 0.30, (m, ratios[m])
    assert ratios[1024] < 1.0


@pytest.mark.parametrize("B,H,Hkv,D,N,bits,m", [(2, 8, 2, 128, 300, 4, 64), (1, 4, 4, 64, 700, 3, 96),
                                               (1, 16, 8, 256, 1100, 4, 1024),
                                               # Gemma 4 full attention (turboquant.rs:1638-1650):
                                               # 16 heads a KV head at D = 512
                                               (1, 32, 2, 512, 700, 4, 64),
                                               (2, 32, 2, 128, 300, 3, 32)])
def test_codebook_decode_with_qjl(T, B, H, Hkv, D, N, bits, m):
    print(f"[qjl-decode] B={B} H={H}/{Hkv} D={D} N={N} bits={bits} m={m}", flush=True)
    R, phi = T.rotation_matrix(D, 42), T.qjl_matrix(D, m, 43)
    b, c = T.lloyd_max(bits)
    cf = c.astype(np.float32)
    rows = B * Hkv * N
    W = (m + 31) // 32
    k = kv_bf16((B, Hkv, N, D), 5, frac=0.02, mult=8.0)
    v = kv_bf16((B, Hkv, N, D), 6, frac=0.02, mult=8.0)
    dR, dphi = T.DeviceArray.of(R), T.DeviceArray.of(phi)
    db, dc = T.DeviceArray.of(b), T.DeviceArray.of(cf)
    bufs = {}
    for name, x, mm in (("k", k, m), ("v", v, 0)):
        codes = T.DeviceArray((rows, D), np.uint8)
        sig = T.DeviceArray((rows,), np.float32)
        sg = T.DeviceArray((rows, max(W, 1)), np.uint32, np.zeros((rows, max(W, 1)), np.uint32))
        rn = T.DeviceArray((rows,), np.float32, np.zeros(rows, np.float32))
        dx = T.DeviceArray.of(x)
        T.tq_encode(dx.ptr, True, 1, rows, D, dR.ptr, db.ptr, dc.ptr, bits, dphi.ptr, mm,
                    codes.ptr, sig.ptr, sg.ptr, rn.ptr)
        bufs[name] = (codes, sig, sg, rn)
    q = kv_bf16((B, H, 1, D), 9)
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    kc, ks, ksg, krn = bufs["k"]
    vc, vs, _, _ = bufs["v"]
    import ctypes
    rc = T.lib().tqkv_decode_attend_codebook_qjl(
        dq.ptr, B, H, Hkv, D, D ** -0.5, dR.ptr, dc.ptr, bits, dc.ptr, bits, kc.ptr, ks.ptr,
        ksg.ptr, krn.ptr, dphi.ptr, m, vc.ptr, vs.ptr, N, N, out.ptr, None, 0, None)
    T.check(rc)
    T.hip().sync()
    sh = lambda a, *t: a.reshape(B, Hkv, N, *t)
    want = O.attend_codebook_qjl(q, sh(kc.numpy(), D), sh(ks.numpy()), sh(ksg.numpy(), W),
                                 sh(krn.numpy()), sh(vc.numpy(), D), sh(vs.numpy()), cf, cf, R,
                                 phi, m, D ** -0.5)
    check_bf16(out.numpy().reshape(B, H, D), want, "qjl-decode")
