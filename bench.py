"""Quantized-KV decode benchmark (the headline).

One step = quantize-on-append of one new K and V token for every sequence
(MLX affine, 3-bit, group 64) followed by fused decode attention over the
whole cache: B=32 sequences, 16 query / 8 KV heads, head_dim 256, 32,768
cached tokens per sequence. Inputs are synthetic (seeded N(0,1) with 1% of
channels x10, generated on the device) and resident in HBM before timing.

Timing: 128 whole steps run untimed first (--settle; from idle the GPU's
clocks take 10-30 ms of load to settle, and per-launch times fall from ~550 µs
to ~305 µs over that span), then the W warm-up steps, then the K timed steps.
"settle_steps" reports how many ran.

Prints one JSON line: value = decode tokens/s (B / step time); the roofline
block prices the decode kernel's algorithmic bytes (packed K/V codes, scales
and biases of the live context, plus Q in and O out) per launch against the
launch duration measured with HIP events on the stream it runs on. The CPU
baseline times the oracle's dequantize-then-attend (the reference semantics
restated in C++) on a bounded sample of the same cache.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "lumen-rs_amd"))

METRIC = "quantized-KV decode attn achieved HBM GB/s + tokens/s @ B=32, 32K ctx"
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 50; the config workloads use their config's "
                         "own step count: decode1 256, prefix 128, layers --decode-steps)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle", type=int, default=None,
                    help="untimed steps before the warm-up (default: 128 decode steps, "
                         "~40 ms; 16 prefill launches): from idle the clocks take 10-30 ms "
                         "of load to reach their loaded state")
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU time budget for the baseline sample")
    ap.add_argument("--workload", choices=("decode", "prefill", "append", "decode1", "prefix",
                                           "layers", "sparse", "codebook"), default="decode",
                    help="decode: config 2 (the headline); prefill: config 3's 2048-token "
                         "chunk attention; append: config 0's quantize round trip (affine, "
                         "affine+rotation, TurboQuant codebook); decode1: config 1's "
                         "single-sequence decode; layers: config 3's 30-layer stack (chunked "
                         "prefill, then decode steps); prefix: config 4's shared-prefix decode; "
                         "sparse: config 2's shape with page-sparse decode; codebook: config "
                         "2's shape over a TurboQuant codebook cache")
    ap.add_argument("--two-launch", action="store_true",
                    help="decode steps append with the quantize kernel and then attend (two "
                         "launches) instead of the decode kernel quantizing the new token "
                         "itself (tqkv_decode_attend_affine_append / tqkv_cache_append_decode)")
    ap.add_argument("--decode-steps", type=int, default=512,
                    help="decode steps of the layers workload (config 3: 512)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(how the path shards over GPUs is a written design, not built)"}))
        sys.exit(2)

    if args.steps is None and args.workload in ("decode", "prefill", "append"):
        args.steps = 50

    import tqkv as T

    hip = T.hip()
    hip._ok(hip.h.hipSetDevice(0), "hipSetDevice")
    others = {"prefill": prefill_main, "append": append_main, "decode1": decode1_main,
              "prefix": prefix_main, "layers": layers_main, "sparse": sparse_main,
              "codebook": codebook_main}
    if args.workload in others:
        others[args.workload](T, hip, args)
        return
    B, H, HKV, D, N, GS, BITS = args.batch, 16, 8, 256, args.context, 64, 3
    scale = D ** -0.5
    steps, warmup = args.steps, args.warmup
    settle = 128 if args.settle is None else max(0, args.settle)
    cap = (N + settle + warmup + steps + 255) // 256 * 256
    words, groups = D * BITS // 32, D // GS
    slabs = B * HKV

    stream = hip.stream()
    cache = {}
    for name in ("k", "v"):
        cache[name] = (T.DeviceArray((slabs, cap, words), np.uint32),
                       T.DeviceArray((slabs, cap, groups), np.uint16),
                       T.DeviceArray((slabs, cap, groups), np.uint16))

    # Fill the first N tokens: synthesize bf16 K/V chunks on the device and
    # quantize them into place with the append kernel.
    chunk = 1024
    tmp = T.DeviceArray((slabs, chunk, D), np.uint16)
    for name, seed in (("k", 11), ("v", 22)):
        pk, sc, bi = cache[name]
        for c0 in range(0, N, chunk):
            n = min(chunk, N - c0)
            T.synth_bf16(tmp.ptr, slabs * n, D, seed * 1000003 + c0, 0.01, 10.0, stream)
            T.affine_quantize(tmp.ptr, slabs, n, D, GS, BITS, pk.ptr, sc.ptr, bi.ptr, cap, c0,
                              stream)
    del tmp
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    T.synth_bf16(q.ptr, B * H, D, 33, 0.0, 1.0, stream)
    newk = T.DeviceArray((slabs, 1, D), np.uint16)
    newv = T.DeviceArray((slabs, 1, D), np.uint16)
    T.synth_bf16(newk.ptr, slabs, D, 44, 0.01, 10.0, stream)
    T.synth_bf16(newv.ptr, slabs, D, 55, 0.01, 10.0, stream)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    ws_bytes = T.decode_workspace_size(B, H, HKV, D, cap)
    ws = T.DeviceArray((ws_bytes,), np.uint8, np.zeros(ws_bytes, np.uint8))
    hip.sync()

    kp = tuple(a.ptr for a in cache["k"])
    vp = tuple(a.ptr for a in cache["v"])
    ev = [(hip.event(), hip.event()) for _ in range(steps)]

    fused = not args.two_launch

    def step(i, events=None):
        pos = N + i  # the new token's row
        if fused:  # the decode kernel quantizes the new token into row pos itself
            seg = T.affine_seg(kp, vp, cap, pos)
            if events:
                hip.record(events[0], stream)
            T.decode_attend_affine_append(q.ptr, B, H, HKV, D, GS, BITS, BITS, scale, [seg],
                                          newk.ptr, newv.ptr, kp + vp, cap, pos, out.ptr,
                                          ws.ptr, ws_bytes, stream)
            if events:
                hip.record(events[1], stream)
            return
        T.affine_quantize_kv(newk.ptr, newv.ptr, slabs, 1, D, GS, BITS, BITS, kp, vp, cap, pos,
                             stream)
        seg = T.affine_seg(kp, vp, cap, pos + 1)
        if events:
            hip.record(events[0], stream)
        T.decode_attend_affine(q.ptr, B, H, HKV, D, GS, BITS, BITS, scale, [seg], out.ptr,
                               ws.ptr, ws_bytes, stream)
        if events:
            hip.record(events[1], stream)

    # Clock settling (untimed whole steps), then the W warm-up steps, then
    # the K timed ones.
    for i in range(settle):
        step(i)
    for i in range(warmup):
        step(settle + i)
    hip._ok(hip.h.hipStreamSynchronize(stream), "sync")
    # The K timed steps, one event pair around all of them (the throughput).
    t0, t1 = hip.event(), hip.event()
    hip.record(t0, stream)
    wall0 = time.perf_counter()
    for i in range(steps):
        step(settle + warmup + i)
    hip.record(t1, stream)
    total_ms = hip.elapsed_ms(t0, t1)
    wall = time.perf_counter() - wall0
    # The same K steps again (same rows rewritten with the same tokens), each
    # decode launch bracketed by events: the kernel's launch duration.
    for i in range(steps):
        step(settle + warmup + i, ev[i])
    hip.sync()
    dec_ms = [hip.elapsed_ms(a, b) for a, b in ev]
    dec_avg_ms = float(np.mean(dec_ms))

    row_bytes = words * 4 + 2 * groups * 2  # packed codes + bf16 scales + bf16 biases
    ctx_avg = N + settle + warmup + (steps - 1) / 2.0 + 1
    alg_bytes = 2 * slabs * ctx_avg * row_bytes + 2 * B * H * D * 2  # K+V, then Q in + O out
    if fused:  # the launch also reads the new bf16 rows and writes their codes
        alg_bytes += 2 * slabs * (D * 2 + row_bytes)
    achieved = alg_bytes / (dec_avg_ms * 1e-3) / 1e9
    ms_per_step = total_ms / steps
    # HBM bytes per decode launch: the two counter passes recorded in
    # profiles/decode_affine_config2.md over the default command's 50 timed
    # launches (FETCH_SIZE 922,781.7 KiB x 2.000 + WRITE_SIZE 336.0 KiB x
    # 1.000, the factors a 1 GiB read and a 1 GiB write kernel of the same
    # library give) = 1,890,201,014 B against 1,888,980,992 B algorithmic
    # (the launch quantizing the new token): 1.000646 per algorithmic byte.
    # Counters cannot be read inside this process; other step counts of the
    # same config scale by that ratio (the context differs by a few tokens),
    # other configs and the two-launch step report null.
    kind = T.decode_kernel_name(H, HKV, D, GS, BITS, BITS)
    kernel = ("decode_mfma_kernel<256,3,3,2,4,8>" if kind == "mfma"
              else "decode_affine_kernel<256,3,3,2,32,8>")
    default_shape = (B, N) == (32, 32768)
    traffic = (int(alg_bytes * 1.000646) if default_shape and kind == "mfma" and fused
               else None)
    tokens_per_s = B / (ms_per_step * 1e-3)

    # Sanity of the result itself: finite, not all zero.
    o = T.bf16_to_f32(out.numpy()) if hasattr(T, "bf16_to_f32") else None
    if o is None:
        o = (out.numpy().astype(np.uint32) << 16).view(np.float32)
    assert np.all(np.isfinite(o)) and np.abs(o).max() > 0, "decode output is not sane"

    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "settle_steps": settle,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 in/out, f16 operands, f32 accumulate",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 2: batched decode over a 3-bit affine cache "
                        "(append 1 token + fused decode attention per step" +
                        (", one launch: the decode kernel quantizes the new token)" if fused
                         else ", two launches)"),
            "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "context": N,
            "bits_k": BITS, "bits_v": BITS, "group_size": GS,
            "layers": 1,
        },
        "hbm_gbps": round(achieved, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": ("profile-derived, not counted in this run: the FETCH_SIZE x 2.000 + "
                               "WRITE_SIZE counter passes of profiles/decode_affine_config2.md "
                               "give 1.000646 HBM bytes per algorithmic byte, applied to this "
                               "run's algorithmic bytes" if traffic is not None else None),
            "kernel": kernel,
            "alg_bytes_per_launch": int(alg_bytes),
            "avg_launch_ms": round(dec_avg_ms, 5),
        },
        "host_wall_ms_per_step": round(wall / steps * 1e3, 4),
    }
    probe = T.measure_read_bandwidth(stream)
    result["read_probe"] = probe
    result["roofline"]["frac_of_read_probe"] = round(achieved / probe["median_gbps"], 4)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(T, cache, q, out, B, H, HKV, D, N, GS, BITS,
                                              scale, cap, args.cpu_seconds)
    print(json.dumps(result))


def cpu_baseline(T, cache, q, out, B, H, HKV, D, N, GS, BITS, scale, cap, budget_s):
    """The reference's decode semantics as an f32 CPU port (dequantize
    exactly, f32 scores / softmax / weighted sum, bf16 out; OpenMP over
    (sequence, KV head)) on whole sequences of the same cache: sequence 0 at
    one thread, and enough sequences for every thread at the box's thread
    count."""
    O, threads = _oracle()
    n_seq = max(1, min(B, -(-2 * threads // HKV)))
    qh = q.numpy()
    kt = tuple(T.hip().download(a.ptr, (n_seq, HKV, cap, a.shape[-1]), a.dtype)
               for a in cache["k"])
    vt = tuple(T.hip().download(a.ptr, (n_seq, HKV, cap, a.shape[-1]), a.dtype)
               for a in cache["v"])

    def run(n, th):
        return lambda: O.attend_affine_f32(qh[:n], tuple(a[:n] for a in kt),
                                           tuple(a[:n] for a in vt), N, GS, BITS, BITS, scale,
                                           threads=th)

    return _port_baseline(run(1, 1), 1, run(n_seq, threads), n_seq, threads, budget_s,
                          f"decode steps over the benchmark's own cache, {HKV} KV heads x {N} "
                          f"tokens a sequence: sequence 0 at 1 thread, sequences 0-{n_seq - 1} "
                          f"at {threads} threads")


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _port_baseline(fn1, tok1, fnn, tokn, threads, budget_s, sample):
    """Median time of fn1 (1 thread, tok1 tokens a call) and fnn (`threads`
    threads, tokn tokens a call) after one warm-up call each, as many timed
    calls (3 to 10) as fit about half the budget each; value = tokens/s at
    `threads` threads, single_thread beside it."""
    def med(fn):
        t = time.perf_counter()
        fn()
        first = time.perf_counter() - t
        reps = int(max(3, min(10, 0.5 * budget_s / max(first, 1e-3))))
        times = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
        return float(np.median(times)), reps

    t1, r1 = med(fn1)
    tn, rn = med(fnn)
    return {
        "value": round(tokn / tn, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": sample + f"; f32 dequantize-then-attend (the oracle library's CPU port of "
                           f"the reference's semantics), median of {r1} / {rn} calls after a "
                           f"warm-up",
        "single_thread": {"value": round(tok1 / t1, 3), "unit": "tokens/s", "cores": 1,
                          "s_per_call": round(t1, 4)},
        "s_per_call": round(tn, 4),
        "cpu_model": _cpu_model(),
        "cpus_visible": os.cpu_count(),
    }


PEAK_BF16_TFLOPS = 2500.0
PREFILL_METRIC = "quantized-KV prefill chunk attention tokens/s (MFMA)"


def visible_pairs(L, N, q_start, k_start, window):
    """(query row, key) pairs the absolute-position mask lets through."""
    qa = q_start + np.arange(L, dtype=np.int64)
    lo = np.full(L, k_start, np.int64) if window < 0 else np.maximum(k_start, qa - window + 1)
    hi = np.minimum(qa, k_start + N - 1)
    return int(np.maximum(hi - lo + 1, 0).sum())


def prefill_main(T, hip, args):
    """BASELINE config 3's prefill: 2048-token chunks over a 4-bit gs64
    cache, B=4, 32 query / 8 KV heads, D=128, scale 1.0 (Gemma). The timed
    step is one chunk attention of a global layer at its last chunk (16,384
    keys, causal); the sliding layer's chunk (3,071 held keys, window 1024)
    is reported beside it. Algorithmic FLOPs = 4 * D * visible (row, key)
    pairs per head (QK^T and PV)."""
    B, H, HKV, D, L, GS, BITS = 4, 32, 8, 128, 2048, 64, 4
    N_G, N_L, W = 16384, 1023 + 2048, 1024
    stream = hip.stream()
    slabs, words, groups = B * HKV, D * BITS // 32, D // GS

    def cache(N, seed):
        trip = {}
        tmp = T.DeviceArray((slabs, 1024, D), np.uint16)
        for name, sd in (("k", seed), ("v", seed + 1)):
            t3 = (T.DeviceArray((slabs, N, words), np.uint32),
                  T.DeviceArray((slabs, N, groups), np.uint16),
                  T.DeviceArray((slabs, N, groups), np.uint16))
            for c0 in range(0, N, 1024):
                n = min(1024, N - c0)
                T.synth_bf16(tmp.ptr, slabs * n, D, sd * 1000003 + c0, 0.01, 10.0, stream)
                T.affine_quantize(tmp.ptr, slabs, n, D, GS, BITS, *(a.ptr for a in t3), N, c0,
                                  stream)
            trip[name] = t3
        return trip

    cg, cl = cache(N_G, 11), cache(N_L, 21)
    q = T.DeviceArray((B, H, L, D), np.uint16)
    T.synth_bf16(q.ptr, B * H * L, D, 33, 0.0, 1.0, stream)
    out = T.DeviceArray((B, H, L, D), np.uint16)
    seg_g = T.affine_seg(tuple(a.ptr for a in cg["k"]), tuple(a.ptr for a in cg["v"]), N_G, N_G)
    seg_l = T.affine_seg(tuple(a.ptr for a in cl["k"]), tuple(a.ptr for a in cl["v"]), N_L, N_L)
    qs_g, ks_g = N_G - L, 0                 # last chunk of a 16,384-token prompt
    qs_l, ks_l = N_G - L, N_G - N_L         # the ring's view: newest 1023 + the chunk

    def run(seg, qs, ks, win):
        T.prefill_attend_affine(q.ptr, B, H, HKV, L, D, GS, BITS, BITS, 1.0, [seg], out.ptr,
                                qs, ks, True, win, stream)

    def timed(seg, qs, ks, win, n):
        evs = [(hip.event(), hip.event()) for _ in range(n)]
        for a, b in evs:
            hip.record(a, stream)
            run(seg, qs, ks, win)
            hip.record(b, stream)
        hip.sync()
        return [hip.elapsed_ms(a, b) for a, b in evs]

    settle = 16 if args.settle is None else max(0, args.settle)
    for _ in range(settle):
        run(seg_g, qs_g, ks_g, -1)
    for _ in range(args.warmup):
        run(seg_g, qs_g, ks_g, -1)
    hip.sync()
    t0, t1 = hip.event(), hip.event()
    hip.record(t0, stream)
    for _ in range(args.steps):
        run(seg_g, qs_g, ks_g, -1)
    hip.record(t1, stream)
    total_ms = hip.elapsed_ms(t0, t1)
    ms_g = float(np.mean(timed(seg_g, qs_g, ks_g, -1, max(3, args.steps // 4))))
    ms_l = float(np.mean(timed(seg_l, qs_l, ks_l, W, max(3, args.steps // 4))))
    fl_g = 4.0 * D * visible_pairs(L, N_G, qs_g, ks_g, -1) * B * H
    fl_l = 4.0 * D * visible_pairs(L, N_L, qs_l, ks_l, W) * B * H
    tf_g = fl_g / (ms_g * 1e-3) / 1e12
    ms_per_step = total_ms / args.steps
    o = (out.numpy().astype(np.uint32) << 16).view(np.float32)
    assert np.all(np.isfinite(o)) and np.abs(o).max() > 0, "prefill output is not sane"
    # HBM bytes of one global-chunk call at this shape, from the FETCH_SIZE
    # (x 2.000) and WRITE_SIZE (x 1.000) passes of
    # profiles/prefill_affine_config3.md: dequantize-once 75.55 MB read +
    # 268.44 MB written, attention 335.88 MB read + 67.11 MB written.
    traffic = 746973184 if (B, L, N_G) == (4, 2048, 16384) else None
    result = {
        "metric": PREFILL_METRIC,
        "value": round(B * L / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "settle_steps": settle,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 in/out, bf16 Q K^T, f16 P V, f32 accumulate", "data": "synthetic",
        "config": {
            "workload": "BASELINE config 3: one 2048-token prefill chunk attention of a "
                        "global layer at 16,384 keys (causal), over a 4-bit gs64 cache",
            "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "chunk": L,
            "keys": N_G, "bits_k": BITS, "bits_v": BITS, "group_size": GS,
        },
        "roofline": {
            "bound": "mfma", "achieved": round(tf_g, 1), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf_g / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
            "traffic_source": ("profile-derived, not counted in this run: the counter passes "
                               "of profiles/prefill_affine_config3.md (both launches of the "
                               "call)" if traffic is not None else None),
            "kernel": "tqkv_prefill_attend_affine call: dequantize_rows_kernel<128,4> (the "
                      "keys once: K bf16 rows, V f16 operands as transposed 64-key tiles) + "
                      "prefill_affine_kernel<128,16,18>",
            "alg_flops_per_launch": fl_g, "avg_launch_ms": round(ms_g, 5),
        },
        "sliding_layer_chunk": {
            "keys": N_L, "window": W, "avg_launch_ms": round(ms_l, 5),
            "tflops": round(fl_l / (ms_l * 1e-3) / 1e12, 1),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = prefill_cpu_baseline(T, cg, q, B, H, HKV, D, L, N_G, GS, BITS,
                                                      qs_g)
    print(json.dumps(result))


def prefill_cpu_baseline(T, cg, q, B, H, HKV, D, L, N, GS, BITS, q_start):
    """The f32 CPU port of dequantize(bf16)-then-attend on the chunk's last
    32 query rows (all heads, all keys): batch row 0 at one thread, every
    batch row at the box's thread count; tokens/s = rows / time."""
    O, threads = _oracle()
    rows = 32
    qh = np.ascontiguousarray(q.numpy()[:, :, L - rows:])
    kt = tuple(np.ascontiguousarray(a.numpy().reshape(B, HKV, N, -1)) for a in cg["k"])
    vt = tuple(np.ascontiguousarray(a.numpy().reshape(B, HKV, N, -1)) for a in cg["v"])

    def run(n, th):
        return lambda: O.attend_affine_f32(qh[:n], tuple(a[:n] for a in kt),
                                           tuple(a[:n] for a in vt), N, GS, BITS, BITS, 1.0,
                                           threads=th, causal=True, q_start=q_start + L - rows,
                                           first_held=0, dequant="bf16")

    return _port_baseline(run(1, 1), rows, run(B, threads), B * rows, threads, 12.0,
                          f"the last {rows} query rows of the chunk, {H} heads x {N} keys: batch "
                          f"row 0 at 1 thread, all {B} batch rows at {threads} threads")


# ------------------------------------------------------------ other configs
def _loop_ms(hip, stream, fn, n):
    """Milliseconds per call of n back-to-back calls of fn, timed by one
    event pair around the whole loop (events between calls cost the stream
    a few microseconds each, which per-call brackets would count)."""
    t0, t1 = hip.event(), hip.event()
    hip.record(t0, stream)
    for _ in range(n):
        fn()
    hip.record(t1, stream)
    hip.sync()
    return hip.elapsed_ms(t0, t1) / n


def _launch_floor_us(T, hip, stream, n=400):
    """Microseconds per launch of n back-to-back empty kernels of 256
    workgroups on `stream`: the floor every launch of a latency-bound step
    pays whatever it does."""
    T.empty_launch(256, stream)
    hip.sync()
    return round(_loop_ms(hip, stream, lambda: T.empty_launch(256, stream), n) * 1e3, 3)


def _line(metric, value, unit, ms, args, dtype, config, roofline, extra=None, settle=0,
          steps=None):
    """One result line; `steps` is the count actually timed (the workloads
    that follow a BASELINE config's own step count pass it)."""
    out = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1,
           "steps": args.steps if steps is None else steps, "warmup": args.warmup,
           "settle_steps": settle,
           "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config,
           "roofline": roofline}
    if extra:
        out.update(extra)
    return out


def _hbm(achieved, kernel, alg, ms, traffic=None):
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": kernel,
            "alg_bytes_per_launch": int(alg), "avg_launch_ms": round(ms, 5)}


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    return O, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def append_main(T, hip, args):
    """one layer's append-quantize round trip, B=1, 8 KV
    heads, D=128, 4,096 tokens, bf16 N(0,1) with 2% of channels x8, 4-bit
    gs64, seed-42 rotation. Timed: quantize K and V (mlx affine), the
    dequantize back, the affine+rotation mode (K rotated by R, then K and V
    quantized, one launch; gemma4_moe.rs:4154-4173) and the TurboQuant codebook encode
    (compress_one, QJL m=64). value = tokens/s of the affine K+V quantize."""
    B, HKV, D, S, GS, BITS, M = 1, 8, 128, 4096, 64, 4, 64
    stream = hip.stream()
    slabs, words, groups = B * HKV, D * BITS // 32, D // GS
    x = {n: T.DeviceArray((slabs, S, D), np.uint16) for n in ("k", "v")}
    T.synth_bf16(x["k"].ptr, slabs * S, D, 101, 0.02, 8.0, stream)
    T.synth_bf16(x["v"].ptr, slabs * S, D, 102, 0.02, 8.0, stream)
    q3 = {n: (T.DeviceArray((slabs, S, words), np.uint32), T.DeviceArray((slabs, S, groups), np.uint16),
              T.DeviceArray((slabs, S, groups), np.uint16)) for n in ("k", "v")}
    deq = {n: T.DeviceArray((slabs, S, D), np.uint16) for n in ("k", "v")}
    rot = {n: T.DeviceArray((slabs, S, D), np.uint16) for n in ("k", "v")}
    R = T.DeviceArray.of(T.rotation_matrix(D, 42))
    bnd, cen = T.lloyd_max(BITS)
    dbnd, dcen = T.DeviceArray.of(bnd), T.DeviceArray.of(cen.astype(np.float32))
    phi = T.DeviceArray.of(T.qjl_matrix(D, M, 43))
    codes = {n: T.DeviceArray((slabs, S, D), np.uint8) for n in ("k", "v")}
    sig = {n: T.DeviceArray((slabs, S), np.float32) for n in ("k", "v")}
    sgn = {n: T.DeviceArray((slabs, S, M // 32), np.uint32) for n in ("k", "v")}
    rn = {n: T.DeviceArray((slabs, S), np.float32) for n in ("k", "v")}

    def quant():  # K and V in one launch, as a cache append issues them
        T.affine_quantize_kv(x["k"].ptr, x["v"].ptr, slabs, S, D, GS, BITS, BITS,
                             tuple(a.ptr for a in q3["k"]), tuple(a.ptr for a in q3["v"]),
                             stream=stream)

    def dequant():
        for n in ("k", "v"):
            T.affine_dequantize(*(a.ptr for a in q3[n]), slabs * S, D, GS, BITS, deq[n].ptr, stream)

    def rotq():  # the affine + rotation mode: K rotated and quantized, V quantized, one launch
        T.affine_quantize_kv_rotated(x["k"].ptr, x["v"].ptr, slabs, S, D, GS, BITS, BITS, R.ptr,
                                     tuple(a.ptr for a in q3["k"]), tuple(a.ptr for a in q3["v"]),
                                     stream=stream)

    def rotq_k():  # the rotate-and-quantize of K alone (the rotation's FLOPs)
        T.affine_quantize_rotated(x["k"].ptr, slabs, S, D, GS, BITS, R.ptr,
                                  *(a.ptr for a in q3["k"]), stream=stream)

    def rotq_two():  # the same with the VALU rotation kernel, then the K+V quantize
        T.rotate_bf16(x["k"].ptr, slabs * S, D, R.ptr, False, rot["k"].ptr, stream)
        T.affine_quantize_kv(rot["k"].ptr, x["v"].ptr, slabs, S, D, GS, BITS, BITS,
                             tuple(a.ptr for a in q3["k"]), tuple(a.ptr for a in q3["v"]),
                             stream=stream)

    def tq():
        for n in ("k", "v"):
            T.tq_encode(x[n].ptr, True, slabs, S, D, R.ptr, dbnd.ptr, dcen.ptr, BITS, phi.ptr, M,
                        codes[n].ptr, sig[n].ptr, sgn[n].ptr, rn[n].ptr, stream=stream)

    # The reference GPU cache's encode (mode 1: y = bf16(x R), its default
    # for K and V), the codebook rows back to bf16 (the codebook cache's
    # prefill), and the codes packed into stage1_packed u64 words.
    inner = T.DeviceArray.of(np.asarray(bnd[1:-1]).astype(np.float32))
    pw = T.packed_words(D, BITS)
    packed = {n: T.DeviceArray((slabs * S, pw), np.uint64) for n in ("k", "v")}

    def tq_gpu():
        for n in ("k", "v"):
            T.tq_encode_gpu_path(x[n].ptr, slabs, S, D, R.ptr, 1, False, inner.ptr, BITS,
                                 codes[n].ptr, sig[n].ptr, stream=stream)

    def cb_deq():
        for n in ("k", "v"):
            T.codebook_dequantize(codes[n].ptr, sig[n].ptr, dcen.ptr, BITS, slabs * S, D,
                                  deq[n].ptr, stream)

    def pack():
        for n in ("k", "v"):
            T.pack_codes(codes[n].ptr, slabs * S, D, BITS, packed[n].ptr, stream)

    # QJL stage 2 of the keys on the device (qjl_encode_stage2_packed and
    # qjl_apply_correction_packed): residual signs of K against a bf16
    # reconstruction (here the affine dequantize's rows), then K_eff.
    def qjl_enc():
        T.qjl_encode_stage2(x["k"].ptr, deq["k"].ptr, phi.ptr, slabs * S, D, M, sgn["k"].ptr,
                            rn["k"].ptr, stream)

    def qjl_fix():
        T.qjl_apply_correction(deq["k"].ptr, sgn["k"].ptr, rn["k"].ptr, phi.ptr, slabs * S, D, M,
                               rot["v"].ptr, stream)

    settle = 16 if args.settle is None else max(0, args.settle)
    for _ in range(settle + args.warmup):
        quant(), dequant(), rotq(), rotq_k(), rotq_two(), tq(), tq_gpu(), cb_deq(), pack()
        qjl_enc(), qjl_fix()
    hip.sync()
    n = args.steps
    ms_q = _loop_ms(hip, stream, quant, n)
    ms_d = _loop_ms(hip, stream, dequant, n)
    ms_r = _loop_ms(hip, stream, rotq, n)
    ms_rk = _loop_ms(hip, stream, rotq_k, n)
    ms_r2 = _loop_ms(hip, stream, rotq_two, n)
    rot_flop = 2 * slabs * S * D * D  # K only: V is not rotated (gemma4_moe.rs:4154-4173)
    ms_t = _loop_ms(hip, stream, tq, max(3, n // 5))
    ms_g = _loop_ms(hip, stream, tq_gpu, n)
    ms_c = _loop_ms(hip, stream, cb_deq, n)
    ms_p = _loop_ms(hip, stream, pack, n)
    ms_je = _loop_ms(hip, stream, qjl_enc, n)
    ms_jf = _loop_ms(hip, stream, qjl_fix, n)
    sg_bytes = slabs * S * (M // 8 + 4)  # sign words + residual norm, keys
    je_bytes = 2 * slabs * S * D * 2 + sg_bytes
    jf_bytes = 2 * slabs * S * D * 2 + sg_bytes
    cb_bytes = 2 * slabs * S * (D + 4)  # u8 codes + f32 sigma, K and V
    # The KVCache trait object (SimpleCache semantics over the device):
    # host f32 vectors in and out, so these times include the copies across
    # PCIe and the call's synchronization. One head of the layer.
    kvc = T.KVCache(D, bits=BITS, qjl_m=M, seed=42)
    kf = (x["k"].numpy()[0].astype(np.uint32) << 16).view(np.float32)
    vf = (x["v"].numpy()[0].astype(np.uint32) << 16).view(np.float32)
    t_s = time.perf_counter()
    kvc.store(0, 0, kf, vf)
    kv_store_s = time.perf_counter() - t_s
    qv = kf[7] * np.float32(0.5)
    kvc.attend_keys(0, 0, qv)
    reps = 20
    t_s = time.perf_counter()
    for _ in range(reps):
        scv = kvc.attend_keys(0, 0, qv)
    kv_keys_us = (time.perf_counter() - t_s) / reps * 1e6
    wv = np.exp(scv - scv.max()).astype(np.float32)
    wv /= wv.sum()
    kvc.attend_values(0, 0, wv)
    t_s = time.perf_counter()
    for _ in range(reps):
        kvc.attend_values(0, 0, wv)
    kv_values_us = (time.perf_counter() - t_s) / reps * 1e6
    kvc.close()
    pk_bytes = 2 * slabs * S * (D + pw * 8)
    in_bytes = 2 * slabs * S * D * 2
    q_bytes = 2 * slabs * S * (words * 4 + 2 * groups * 2)
    tq_bytes = 2 * slabs * S * (D + 4 + M // 8 + 4)
    result = _line(
        "append-quantize round trip tokens/s (one layer, K and V)", S / (ms_q * 1e-3), "tokens/s",
        ms_q, args, "bf16->u32",
        {"workload": "BASELINE config 0: quantize-on-append of one layer's K and V "
                     "(B=1, 8 KV heads, D=128, 4,096 tokens, 4-bit gs64)",
         "batch": B, "kv_heads": HKV, "head_dim": D, "tokens": S, "bits": BITS, "group_size": GS},
        # HBM bytes per launch from the counter passes recorded in
        # profiles/append_quantize_config0.md (FETCH_SIZE 8,237.0 KiB x 2.000
        # + WRITE_SIZE 4,608.0 KiB x 1.000, the read / write kernels'
        # factors) = 1.00429 per algorithmic byte.
        _hbm((in_bytes + q_bytes) / (ms_q * 1e-3) / 1e9,
             "affine_quantize_kernel<128> (K and V in one launch)", in_bytes + q_bytes, ms_q,
             int((in_bytes + q_bytes) * 1.00429)),
        {"dequantize": {"ms": round(ms_d, 5), "gbps": round((q_bytes + in_bytes) / (ms_d * 1e-3) / 1e9, 1)},
         "affine_rotation": {"ms": round(ms_r, 5),
                             "tokens_per_s": round(S / (ms_r * 1e-3), 1),
                             "kernel": "affine_quantize_rot_kernel<128>: K = bf16(x R) "
                                       "(R split exactly into three bf16 parts, "
                                       "v_mfma_f32_16x16x32_bf16, f32 accumulation), "
                                       "quantized in registers; then V quantized; one launch",
                             "rotation_flop": rot_flop,
                             "k_only_ms": round(ms_rk, 5),
                             "k_only_tflops": round(rot_flop / (ms_rk * 1e-3) / 1e12, 1),
                             "k_only_frac_fp32_peak": round(rot_flop / (ms_rk * 1e-3) / 157.3e12, 4),
                             "bytes": in_bytes + q_bytes,
                             "gbps": round((in_bytes + q_bytes) / (ms_r * 1e-3) / 1e9, 1),
                             "two_launch_ms": round(ms_r2, 5),
                             "two_launch": "tqkv_rotate_bf16 (VALU f32, R in LDS) of K, then "
                                           "the K+V quantize"},
         "turboquant_encode": {"ms": round(ms_t, 5), "tokens_per_s": round(S / (ms_t * 1e-3), 1),
                               "bytes": in_bytes + tq_bytes, "qjl_m": M,
                               "note": "compress_one restated bit-exactly: sequential f32 "
                                       "sums, four lanes per vector, R and Phi from LDS; "
                                       "VALU-bound (unfused mul + add)"},
         "turboquant_encode_gpu_path": {
             "ms": round(ms_g, 5), "tokens_per_s": round(S / (ms_g * 1e-3), 1),
             "bytes": in_bytes + cb_bytes,
             "gbps": round((in_bytes + cb_bytes) / (ms_g * 1e-3) / 1e9, 1),
             "note": "tqkv_tq_encode_gpu_path mode 1 (y = bf16(x R), sigma, bf16(y / sigma) "
                     "against f32 inner boundaries), K and V"},
         "codebook_dequantize": {
             "ms": round(ms_c, 5), "bytes": cb_bytes + in_bytes,
             "gbps": round((cb_bytes + in_bytes) / (ms_c * 1e-3) / 1e9, 1),
             "note": "tqkv_codebook_dequantize: bf16(centroid * sigma) rows of K and V"},
         "pack_codes": {
             "ms": round(ms_p, 5), "bytes": pk_bytes,
             "gbps": round(pk_bytes / (ms_p * 1e-3) / 1e9, 1),
             "note": "tqkv_pack_codes: u8 codes of K and V to stage1_packed u64 words"},
         "qjl_stage2": {
             "encode_ms": round(ms_je, 5), "encode_bytes": je_bytes,
             "encode_gbps": round(je_bytes / (ms_je * 1e-3) / 1e9, 1),
             "apply_ms": round(ms_jf, 5), "apply_bytes": jf_bytes,
             "apply_gbps": round(jf_bytes / (ms_jf * 1e-3) / 1e9, 1), "qjl_m": M,
             "note": "tqkv_qjl_encode_stage2 (residual signs and norms of K) and "
                     "tqkv_qjl_apply_correction (K_eff rows), keys only"},
         "kvcache_trait": {
             "store_vectors_per_s": round(S / kv_store_s, 1),
             "attend_keys_us": round(kv_keys_us, 1), "attend_values_us": round(kv_values_us, 1),
             "vectors": S, "qjl_m": M,
             "note": "tqkv_kvcache_store / _attend_keys / _attend_values on one head: host f32 "
                     "in and out, PCIe and the synchronizing return included (host clock)"}},
        settle)
    if not args.no_cpu_baseline:
        O, threads = _oracle()
        kh = x["k"].numpy()
        t = time.perf_counter()
        O.affine_quantize(kh, GS, BITS)
        dt = time.perf_counter() - t
        comp = O.Compressor(D, BITS, M, T.rotation_matrix(D, 42), T.qjl_matrix(D, M, 43))
        sample = (kh[0, :256].astype(np.uint32) << 16).view(np.float32)
        t = time.perf_counter()
        comp.compress(sample)
        dtq = time.perf_counter() - t
        result["cpu_baseline"] = {
            "value": round(S / (2 * dt), 1), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle affine quantize of K ({slabs} heads x {S} tokens, {dt:.3f} s; "
                      f"K+V counted as twice that); TurboQuant compress_one of 256 vectors: "
                      f"{256 / dtq:.0f} vectors/s single-threaded"}
    print(json.dumps(result))


def _fill_affine(T, stream, slabs, N, D, GS, bits, cap, seed, start=0):
    words, groups = D * bits // 32, D // GS
    t3 = (T.DeviceArray((slabs, cap, words), np.uint32), T.DeviceArray((slabs, cap, groups), np.uint16),
          T.DeviceArray((slabs, cap, groups), np.uint16))
    tmp = T.DeviceArray((slabs, 1024, D), np.uint16)
    for c0 in range(0, N, 1024):
        n = min(1024, N - c0)
        T.synth_bf16(tmp.ptr, slabs * n, D, seed * 1000003 + c0, 0.01, 10.0, stream)
        T.affine_quantize(tmp.ptr, slabs, n, D, GS, bits, *(a.ptr for a in t3), cap, start + c0,
                          stream)
    return t3


def decode1_main(T, hip, args):
    """one sequence, 32 query / 8 KV heads, D=128, 4-bit
    gs64, context 8,192; a step appends one K and V token and decodes. The
    decode splits the keys over enough workgroups to fill the chip and
    merges the splits (two launches); the line is latency-bound."""
    B, H, HKV, D, N, GS, BITS = 1, 32, 8, 128, 8192, 64, 4
    stream = hip.stream()
    slabs = B * HKV
    settle = 64 if args.settle is None else max(0, args.settle)
    steps = 256 if args.steps is None else args.steps
    cap = N + settle + args.warmup + steps + 1
    kc = _fill_affine(T, stream, slabs, N, D, GS, BITS, cap, 7)
    vc = _fill_affine(T, stream, slabs, N, D, GS, BITS, cap, 8)
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    T.synth_bf16(q.ptr, B * H, D, 9, 0.0, 1.0, stream)
    nk, nv = T.DeviceArray((slabs, 1, D), np.uint16), T.DeviceArray((slabs, 1, D), np.uint16)
    T.synth_bf16(nk.ptr, slabs, D, 10, 0.02, 8.0, stream)
    T.synth_bf16(nv.ptr, slabs, D, 11, 0.02, 8.0, stream)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    wsb = T.decode_workspace_size(B, H, HKV, D, cap)
    ws = T.DeviceArray((wsb,), np.uint8)
    kp, vp = tuple(a.ptr for a in kc), tuple(a.ptr for a in vc)
    pos = [N]
    fused = not args.two_launch

    def append():
        if fused:  # the decode launch quantizes the token itself
            return
        T.affine_quantize_kv(nk.ptr, nv.ptr, slabs, 1, D, GS, BITS, BITS, kp, vp, cap, pos[0],
                             stream)
        pos[0] += 1

    def decode():
        if fused:
            seg = T.affine_seg(kp, vp, cap, pos[0])
            T.decode_attend_affine_append(q.ptr, B, H, HKV, D, GS, BITS, BITS, D ** -0.5, [seg],
                                          nk.ptr, nv.ptr, kp + vp, cap, pos[0], out.ptr, ws.ptr,
                                          wsb, stream)
            pos[0] += 1
            return
        seg = T.affine_seg(kp, vp, cap, pos[0])
        T.decode_attend_affine(q.ptr, B, H, HKV, D, GS, BITS, BITS, D ** -0.5, [seg], out.ptr,
                               ws.ptr, wsb, stream)

    for _ in range(settle + args.warmup):
        append(), decode()
    hip.sync()
    ctx0 = pos[0]
    step_ms = _loop_ms(hip, stream, lambda: (append(), decode()), steps)
    # The same steps again (rows rewritten with the same tokens), each decode
    # bracketed by events.
    pos[0] = ctx0
    evs = [(hip.event(), hip.event()) for _ in range(steps)]
    for b, c in evs:
        append()
        hip.record(b, stream)
        decode()
        hip.record(c, stream)
    hip.sync()
    dec_ms = float(np.mean([hip.elapsed_ms(b, c) for b, c in evs]))
    row = D * BITS // 32 * 4 + 2 * (D // GS) * 2
    ctx = ctx0 + (steps + 1) / 2.0
    alg = 2 * slabs * ctx * row + 2 * B * H * D * 2
    result = _line(
        "single-sequence quantized-KV decode tokens/s", 1.0 / (step_ms * 1e-3), "tokens/s", step_ms,
        args, "bf16 in/out, f16 operands, f32 accumulate",
        {"workload": "BASELINE config 1: 1 sequence, 32/8 heads, D=128, 4-bit gs64, 8,192 "
                     "context, 256 steps each appending one token",
         "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "context": N, "steps": steps,
         "launches_per_step": 2 if fused else 3},
        _hbm(alg / (dec_ms * 1e-3) / 1e9, T.decode_kernel_name(H, HKV, D, GS, BITS, BITS) +
             (" split (quantizing the new token) + merge" if fused else " split + merge"),
             alg, dec_ms),
        {"decode_us": round(dec_ms * 1e3, 2), "step_us": round(step_ms * 1e3, 2),
         "launch_floor_us": _launch_floor_us(T, hip, stream)}, settle, steps)
    if not args.no_cpu_baseline:
        O, threads = _oracle()
        kt = tuple(a.numpy()[:, :pos[0]].reshape(B, HKV, pos[0], -1) for a in kc)
        vt = tuple(a.numpy()[:, :pos[0]].reshape(B, HKV, pos[0], -1) for a in vc)
        qh = q.numpy()

        def run(th):
            return lambda: O.attend_affine_f32(qh, kt, vt, pos[0], GS, BITS, BITS, D ** -0.5,
                                               threads=th)

        result["cpu_baseline"] = _port_baseline(
            run(1), 1, run(threads), 1, threads, 12.0,
            f"one decode step of the sequence ({pos[0]} keys, {HKV} KV heads)")
    print(json.dumps(result))


def prefix_main(T, hip, args):
    """8 sequences over one shared 65,536-token prefix
    (stored once, batch stride 0) plus 4,096 tokens of their own, 32 query
    / 8 KV heads, D=128, 8-bit keys and 4-bit values, gs64; a step appends
    one token per sequence and decodes over prefix + suffix in one softmax.
    Achieved bandwidth is priced on the unique bytes (the prefix once)."""
    B, H, HKV, D, P, S0, GS, BK, BV = 8, 32, 8, 128, 65536, 4096, 64, 8, 4
    stream = hip.stream()
    settle = 32 if args.settle is None else max(0, args.settle)
    steps = 128 if args.steps is None else args.steps
    cap = S0 + settle + args.warmup + steps + 1
    pk = _fill_affine(T, stream, HKV, P, D, GS, BK, P, 21)
    pv = _fill_affine(T, stream, HKV, P, D, GS, BV, P, 22)
    sk = _fill_affine(T, stream, B * HKV, S0, D, GS, BK, cap, 23)
    sv = _fill_affine(T, stream, B * HKV, S0, D, GS, BV, cap, 24)
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    T.synth_bf16(q.ptr, B * H, D, 25, 0.0, 1.0, stream)
    nk, nv = T.DeviceArray((B * HKV, 1, D), np.uint16), T.DeviceArray((B * HKV, 1, D), np.uint16)
    T.synth_bf16(nk.ptr, B * HKV, D, 26, 0.0, 1.0, stream)
    T.synth_bf16(nv.ptr, B * HKV, D, 27, 0.0, 1.0, stream)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    wsb = T.decode_workspace_size(B, H, HKV, D, P + cap)
    ws = T.DeviceArray((wsb,), np.uint8)
    pkp, pvp = tuple(a.ptr for a in pk), tuple(a.ptr for a in pv)
    skp, svp = tuple(a.ptr for a in sk), tuple(a.ptr for a in sv)
    pos = [S0]

    fused = not args.two_launch

    def step(events=None):
        if fused:  # the suffix decode launch quantizes the token itself
            segs = [T.affine_seg(pkp, pvp, P, P, shared=True),
                    T.affine_seg(skp, svp, cap, pos[0])]
            if events:
                hip.record(events[0], stream)
            T.decode_attend_affine_append(q.ptr, B, H, HKV, D, GS, BK, BV, D ** -0.5, segs,
                                          nk.ptr, nv.ptr, skp + svp, cap, pos[0], out.ptr,
                                          ws.ptr, wsb, stream)
            if events:
                hip.record(events[1], stream)
            pos[0] += 1
            return
        T.affine_quantize_kv(nk.ptr, nv.ptr, B * HKV, 1, D, GS, BK, BV, skp, svp, cap, pos[0],
                             stream)
        pos[0] += 1
        segs = [T.affine_seg(pkp, pvp, P, P, shared=True), T.affine_seg(skp, svp, cap, pos[0])]
        if events:
            hip.record(events[0], stream)
        T.decode_attend_affine(q.ptr, B, H, HKV, D, GS, BK, BV, D ** -0.5, segs, out.ptr, ws.ptr,
                               wsb, stream)
        if events:
            hip.record(events[1], stream)

    for _ in range(settle + args.warmup):
        step()
    hip.sync()
    ctx0 = pos[0]
    total = _loop_ms(hip, stream, step, steps) * steps
    # The same steps again (rows rewritten with the same tokens), each
    # attention call bracketed by events.
    pos[0] = ctx0
    evs = [(hip.event(), hip.event()) for _ in range(steps)]
    for e in evs:
        step(e)
    hip.sync()
    dec_ms = float(np.mean([hip.elapsed_ms(a, b) for a, b in evs]))
    # And with the prefix read once per sequence (the library's
    # TQKV_SHARED_PREFIX=0 switch), for comparison.
    pos[0] = ctx0
    os.environ["TQKV_SHARED_PREFIX"] = "0"
    try:
        per_seq_ms = _loop_ms(hip, stream, step, steps)
    finally:
        del os.environ["TQKV_SHARED_PREFIX"]
    row = (D * BK // 32 * 4 + 2 * (D // GS) * 2) + (D * BV // 32 * 4 + 2 * (D // GS) * 2)  # 208
    ctx = ctx0 + (steps + 1) / 2.0
    unique = P * HKV * row + B * HKV * ctx * row + 2 * B * H * D * 2
    naive = B * HKV * (P + ctx) * row + 2 * B * H * D * 2
    # HBM bytes per call from the FETCH_SIZE (x 2.000) and WRITE_SIZE (x 1.000)
    # passes of profiles/prefix_shared_config4.md at this command's default
    # steps: prefix pass 113.70 MB + suffix decode 59.41 MB + merge 4.99 MB =
    # 178.11 MB against 165.06 MB algorithmic, 1.07903 per algorithmic byte
    # (the excess is the partial results written and read back by the merge).
    traffic = int(unique * 1.07903) if steps == 128 and fused else None
    hbm = _hbm(unique / (dec_ms * 1e-3) / 1e9,
               "shared-prefix decode call: prefix pass (prefill kernel, f16 tiles) + suffix "
               "decode (" + T.decode_kernel_name(H, HKV, D, GS, BK, BV) + ") + merge", unique,
               dec_ms, traffic)
    if traffic is not None:
        hbm["traffic_source"] = ("profile-derived, not counted in this run: the counter passes "
                                 "of profiles/prefix_shared_config4.md give 1.07903 HBM bytes "
                                 "per algorithmic byte")
    result = _line(
        "prefix-shared quantized-KV decode tokens/s", B / (total / steps * 1e-3), "tokens/s",
        total / steps, args, "bf16 in/out, f16 operands, f32 accumulate",
        {"workload": "BASELINE config 4: 8 sequences sharing a 65,536-token prefix plus 4,096 "
                     "own tokens, 32/8 heads, D=128, K 8-bit / V 4-bit gs64, 128 decode steps",
         "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "prefix": P, "suffix": S0,
         "bits_k": BK, "bits_v": BV, "group_size": GS, "launches_per_step": 3 if fused else 4},
        hbm,
        {"naive_bytes_per_step": int(naive),
         "naive_gbps": round(naive / (dec_ms * 1e-3) / 1e9, 1),
         "per_sequence_path_ms_per_step": round(per_seq_ms, 5),
         "launch_floor_us": _launch_floor_us(T, hip, stream)}, settle, steps)
    if not args.no_cpu_baseline:
        O, threads = _oracle()
        n_seq = max(1, min(B, -(-2 * threads // HKV)))
        pre = [a.numpy()[:, :P] for a in (*pk, *pv)]
        suf = [a.numpy()[:n_seq * HKV, :pos[0]] for a in (*sk, *sv)]
        cat = lambda p_, s_: np.concatenate(
            [np.broadcast_to(p_.reshape(1, HKV, P, -1), (n_seq, HKV, P, p_.shape[-1])),
             s_.reshape(n_seq, HKV, pos[0], -1)], axis=2)
        full = [cat(p_, s_) for p_, s_ in zip(pre, suf)]
        kt, vt = tuple(full[:3]), tuple(full[3:])
        qh = q.numpy()

        def run(n, th):
            return lambda: O.attend_affine_f32(qh[:n], tuple(a[:n] for a in kt),
                                               tuple(a[:n] for a in vt), P + pos[0], GS, BK, BV,
                                               D ** -0.5, threads=th)

        result["cpu_baseline"] = _port_baseline(
            run(1, 1), 1, run(n_seq, threads), n_seq, threads, 12.0,
            f"decode steps over prefix + suffix ({P + pos[0]} keys, the prefix read per "
            f"sequence): sequence 0 at 1 thread, sequences 0-{n_seq - 1} at {threads} threads")
    print(json.dumps(result))


def sparse_main(T, hip, args):
    """Config 2's shape (B=32, 16 / 8 heads, D=256, 32,768-token context,
    3-bit gs64) with page-sparse decode (sdpa_page_sparse, the reference's
    LUMEN_SPARSE_DECODE): a step appends one token per sequence (digesting a
    page when one fills) and attends to the keep = max(pages / 8, 64) pages
    whose key bounds score highest, plus the first, the last four and the
    undigested tail. Not the headline metric (it attends to fewer keys):
    reported beside it. Bytes are the ones the sparse call reads: the digest,
    the chosen pages' K and V, the tail, Q and O."""
    B, H, HKV, D, N, GS, BITS = 32, 16, 8, 256, args.context, 64, 3
    stream = hip.stream()
    slabs = B * HKV
    settle = 64 if args.settle is None else max(0, args.settle)
    steps = 50 if args.steps is None else args.steps
    cap = (N + settle + args.warmup + steps + 255) // 256 * 256
    kc = _fill_affine(T, stream, slabs, N, D, GS, BITS, cap, 11)
    vc = _fill_affine(T, stream, slabs, N, D, GS, BITS, cap, 22)
    max_pages = cap // 64
    kmin = T.DeviceArray((slabs, max_pages, D), np.uint16)
    kmax = T.DeviceArray((slabs, max_pages, D), np.uint16)
    kp, vp = tuple(a.ptr for a in kc), tuple(a.ptr for a in vc)
    pages0 = N // 64
    t0, t1 = hip.event(), hip.event()
    hip.record(t0, stream)
    T.page_digest_affine(kp, slabs, cap, D, GS, BITS, 0, pages0, kmin.ptr, kmax.ptr, max_pages,
                         stream)
    hip.record(t1, stream)
    hip.sync()
    digest_ms = hip.elapsed_ms(t0, t1)
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    T.synth_bf16(q.ptr, B * H, D, 33, 0.0, 1.0, stream)
    nk, nv = T.DeviceArray((slabs, 1, D), np.uint16), T.DeviceArray((slabs, 1, D), np.uint16)
    T.synth_bf16(nk.ptr, slabs, D, 44, 0.01, 10.0, stream)
    T.synth_bf16(nv.ptr, slabs, D, 55, 0.01, 10.0, stream)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    keep_max = int(T.sparse_keep_pages(max_pages))
    wsb = T.sparse_workspace_size(B, H, HKV, D, cap, keep_max)
    ws = T.DeviceArray((wsb,), np.uint8)
    pos = [N]
    digested = [pages0]

    def append():
        T.affine_quantize_kv(nk.ptr, nv.ptr, slabs, 1, D, GS, BITS, BITS, kp, vp, cap, pos[0],
                             stream)
        pos[0] += 1
        if pos[0] // 64 > digested[0]:
            T.page_digest_affine(kp, slabs, cap, D, GS, BITS, digested[0], pos[0] // 64, kmin.ptr,
                                 kmax.ptr, max_pages, stream)
            digested[0] = pos[0] // 64

    def attend():
        pages = digested[0]
        seg = T.affine_seg(kp, vp, cap, pos[0])
        T.decode_attend_affine_sparse(q.ptr, B, H, HKV, D, GS, BITS, BITS, D ** -0.5, seg,
                                      kmin.ptr, kmax.ptr, max_pages, pages,
                                      int(T.sparse_keep_pages(pages)), out.ptr, ws.ptr, wsb,
                                      stream=stream)

    for _ in range(settle + args.warmup):
        append(), attend()
    hip.sync()
    ctx0, dig0 = pos[0], digested[0]
    step_ms = _loop_ms(hip, stream, lambda: (append(), attend()), steps)
    pos[0], digested[0] = ctx0, dig0
    evs = [(hip.event(), hip.event()) for _ in range(steps)]
    alg = []
    row = D * BITS // 32 * 4 + 2 * (D // GS) * 2
    for a_, b_ in evs:
        append()
        pages = digested[0]
        keep = int(T.sparse_keep_pages(pages))
        alg.append(slabs * (2 * keep * 64 * row + 2 * (pos[0] - pages * 64) * row +
                            2 * pages * D * 2) + 2 * B * H * D * 2)
        hip.record(a_, stream)
        attend()
        hip.record(b_, stream)
    hip.sync()
    att_ms = float(np.mean([hip.elapsed_ms(a_, b_) for a_, b_ in evs]))
    alg_b = float(np.mean(alg))
    dense_b = 2 * slabs * (ctx0 + steps / 2.0) * row + 2 * B * H * D * 2
    result = _line(
        "page-sparse quantized-KV decode tokens/s @ B=32, 32K ctx", B / (step_ms * 1e-3),
        "tokens/s", step_ms, args, "bf16 in/out, f16 operands, f32 accumulate",
        {"workload": "config 2's shape (B=32, 16/8 heads, D=256, 32K context, 3-bit gs64) with "
                     "page-sparse decode: keep max(pages/8, 64) pages + sink + 4 recent + tail",
         "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "context": N,
         "bits_k": BITS, "bits_v": BITS, "group_size": GS,
         "keep_pages": int(T.sparse_keep_pages(N // 64))},
        _hbm(alg_b / (att_ms * 1e-3) / 1e9,
             "page bounds + select + decode_mfma_kernel<256,3,3,2,4,8,paged>", alg_b, att_ms),
        {"digest_ms_once": round(digest_ms, 4), "dense_bytes_per_step": int(dense_b),
         "dense_equivalent_gbps": round(dense_b / (att_ms * 1e-3) / 1e9, 1)}, settle, steps)
    print(json.dumps(result))


def codebook_main(T, hip, args):
    """Config 2's shape (B=32, 16 / 8 heads, D=256, 32,768-token context) over
    a TurboQuant codebook cache (the GPU TurboQuant caches' attention,
    turboquant.rs:763-923): 3-bit Lloyd-Max codes as one byte each plus an
    f32 sigma a vector, for K and V, stored rotated. A step is one
    tqkv_decode_attend_codebook call (query rotated, attention over
    centroid * sigma, output rotated back). Not the headline metric (a
    different cache format): reported beside it. Bytes: the codes and sigmas
    of K and V, Q, O and R."""
    B, H, HKV, D, N, BITS = 32, 16, 8, 256, args.context, 3
    stream = hip.stream()
    slabs = B * HKV
    settle = 32 if args.settle is None else max(0, args.settle)
    steps = 50 if args.steps is None else args.steps
    rng = np.random.default_rng(7)
    codes = {}
    sigmas = {}
    for name in ("k", "v"):
        c = T.DeviceArray((slabs, N, D), np.uint8)
        one = rng.integers(0, 1 << BITS, size=(N, D), dtype=np.uint8)
        for sl in range(slabs):  # one slab's codes, rolled per slab
            hip.copy_in(c.ptr + sl * N * D, np.roll(one, sl, axis=0))
        codes[name] = c
        sigmas[name] = T.DeviceArray.of(
            rng.uniform(0.5, 2.0, size=(slabs, N)).astype(np.float32))
    cent = T.DeviceArray.of(T.lloyd_max(BITS)[1].astype(np.float32))
    R = T.DeviceArray.of(T.rotation_matrix(D, 42))
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    T.synth_bf16(q.ptr, B * H, D, 33, 0.0, 1.0, stream)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    wsb = T.decode_codebook_workspace_size(B, H, D, N)
    ws = T.DeviceArray((wsb,), np.uint8)

    def call():
        T.decode_attend_codebook(q.ptr, B, H, HKV, D, D ** -0.5, R.ptr, cent.ptr, BITS, cent.ptr,
                                 BITS, codes["k"].ptr, sigmas["k"].ptr, codes["v"].ptr,
                                 sigmas["v"].ptr, N, N, out.ptr, ws.ptr, wsb, stream)

    for _ in range(settle + args.warmup):
        call()
    hip.sync()
    ms = _loop_ms(hip, stream, call, steps)
    o = (out.numpy().astype(np.uint32) << 16).view(np.float32)
    assert np.all(np.isfinite(o)) and np.abs(o).max() > 0, "codebook output is not sane"
    alg = 2 * slabs * N * (D + 4) + 2 * B * H * D * 2 + D * D * 4
    result = _line(
        "codebook-cache decode tokens/s @ B=32, 32K ctx", B / (ms * 1e-3), "tokens/s", ms, args,
        "bf16 in/out, f32 arithmetic",
        {"workload": "config 2's shape (B=32, 16/8 heads, D=256, 32K context) over a TurboQuant "
                     "codebook cache: 3-bit Lloyd-Max codes (u8) + f32 sigma, K and V rotated",
         "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "context": N,
         "bits_k": BITS, "bits_v": BITS},
        _hbm(alg / (ms * 1e-3) / 1e9, "one call: cb_rotate_q_kernel + cb_decode_kernel<256,2,false> + cb_merge_kernel", alg, ms),
        {"workspace_bytes": wsb}, settle, steps)
    print(json.dumps(result))


def layers_main(T, hip, args):
    """BASELINE config 3 end to end through the cache objects: 30 layers
    (global at 5, 11, 17, 23, 29; the rest sliding with a 1,024-token ring,
    keep 0), B=4, 32 / 8 heads, D=128, 4-bit gs64, scale 1. Prefill: a
    16,384-token prompt in 8 chunks of 2,048 (per chunk and layer: append,
    then chunk attention with the layer's mask). Decode: steps appending one
    token per layer and attending; a step = all 30 layers. tokens/s = B /
    step time (the survey's B / sum over 30 layers)."""
    B, H, HKV, D, GS, BITS, L, CH, W = 4, 32, 8, 128, 64, 4, 16384, 2048, 1024
    n_layers = 30
    glob = {5, 11, 17, 23, 29}
    stream = hip.stream()
    slabs = B * HKV
    caches = [T.Cache(T.CACHE_AFFINE, B, HKV, D, D, GS, BITS, BITS, prealloc=True,
                      max_size=0 if i in glob else W, keep=0) for i in range(n_layers)]
    kc, vc = T.DeviceArray((slabs, CH, D), np.uint16), T.DeviceArray((slabs, CH, D), np.uint16)
    qc = T.DeviceArray((B, H, CH, D), np.uint16)
    oc = T.DeviceArray((B, H, CH, D), np.uint16)
    T.synth_bf16(qc.ptr, B * H * CH, D, 5, 0.0, 1.0, stream)

    def prefill():
        for c0 in range(0, L, CH):
            T.synth_bf16(kc.ptr, slabs * CH, D, 1000 + c0, 0.02, 8.0, stream)
            T.synth_bf16(vc.ptr, slabs * CH, D, 2000 + c0, 0.02, 8.0, stream)
            for i, c in enumerate(caches):
                c.append(kc.ptr, vc.ptr, CH, stream)
                c.prefill_attend(qc.ptr, H, CH, 1.0, oc.ptr, window=-1 if i in glob else W,
                                 stream=stream)

    hip.sync()
    t0, t1 = hip.event(), hip.event()
    hip.record(t0, stream)
    prefill()
    hip.record(t1, stream)
    prefill_ms = hip.elapsed_ms(t0, t1)
    nk, nv = T.DeviceArray((slabs, 1, D), np.uint16), T.DeviceArray((slabs, 1, D), np.uint16)
    T.synth_bf16(nk.ptr, slabs, D, 31, 0.02, 8.0, stream)
    T.synth_bf16(nv.ptr, slabs, D, 32, 0.02, 8.0, stream)
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    T.synth_bf16(q.ptr, B * H, D, 33, 0.0, 1.0, stream)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    wsb = T.decode_workspace_size(B, H, HKV, D, L + args.decode_steps + 64)
    ws = T.DeviceArray((wsb,), np.uint8)

    fused = not args.two_launch

    def step():
        for c in caches:
            if fused:  # one decode launch (+ merge) quantizes the token itself
                c.append_decode(nk.ptr, nv.ptr, q.ptr, H, 1.0, out.ptr, ws.ptr, wsb, stream)
            else:
                c.append(nk.ptr, nv.ptr, 1, stream)
                c.decode_attend(q.ptr, H, 1.0, out.ptr, ws.ptr, wsb, stream)

    settle = 16 if args.settle is None else max(0, args.settle)
    for _ in range(settle + args.warmup):
        step()
    hip.sync()
    views0 = [c.state().view for c in caches]
    steps = args.decode_steps if args.steps is None else args.steps
    step_ms = _loop_ms(hip, stream, step, steps)
    views1 = [c.state().view for c in caches]
    row = D * BITS // 32 * 4 + 2 * (D // GS) * 2  # 72
    avg_view = [(a + b) / 2.0 for a, b in zip(views0, views1)]
    alg = sum(2 * slabs * v * row for v in avg_view) + n_layers * 2 * B * H * D * 2
    result = _line(
        "30-layer rotating-window decode tokens/s", B / (step_ms * 1e-3), "tokens/s", step_ms, args,
        "bf16 in/out, f16 operands, f32 accumulate",
        {"workload": "BASELINE config 3: 30 layers (5 global, 25 sliding ring 1024), B=4, "
                     "32/8 heads, D=128, 4-bit gs64; 16,384-token prefill in 2,048 chunks "
                     "(MFMA chunk attention), then decode steps over all layers",
         "batch": B, "q_heads": H, "kv_heads": HKV, "head_dim": D, "layers": n_layers,
         "prompt": L, "chunk": CH, "window": W, "decode_steps": steps,
         "append": "in the decode kernel" if fused else "own launch"},
        _hbm(alg / (step_ms * 1e-3) / 1e9, "30 x (append + decode) per step", alg, step_ms),
        {"prefill_ms": round(prefill_ms, 2),
         "prefill_tokens_per_s": round(B * L / (prefill_ms * 1e-3), 1),
         "decode_bytes_per_step": int(alg),
         "views_at_end": {"global": int(views1[5]), "sliding": int(views1[0])},
         "launch_floor_us": _launch_floor_us(T, hip, stream)}, settle, steps)
    if not args.no_cpu_baseline:
        # A step of batch row 0 = 25 sliding-layer decodes + 5 global ones;
        # one of each is timed over that layer's cache view (its own keys),
        # and the step time is 25 x sliding + 5 x global.
        O, threads = _oracle()
        spec = [(np.uint32, D * BITS // 32), (np.uint16, D // GS), (np.uint16, D // GS)]
        qh = q.numpy()

        def layer_fn(c, n_b, th):
            v = c.buffers()
            t3 = [T.view_slot(v, i, slabs, dt, w).reshape(B, HKV, v.n, w)[:n_b]
                  for i, (dt, w) in enumerate(spec * 2)]
            return lambda: O.attend_affine_f32(qh[:n_b], tuple(t3[:3]), tuple(t3[3:]), v.n, GS,
                                               BITS, BITS, 1.0, threads=th)

        def step_fn(n_b, th):
            fs, fg = layer_fn(caches[0], n_b, th), layer_fn(caches[5], n_b, th)

            def run():
                t = time.perf_counter()
                fs()
                ts = time.perf_counter() - t
                t = time.perf_counter()
                fg()
                tg = time.perf_counter() - t
                return ts, tg
            return run

        def timed(run):
            run()
            ts, tg = zip(*[run() for _ in range(3)])
            return 25 * float(np.median(ts)) + 5 * float(np.median(tg))

        t1, tn = timed(step_fn(1, 1)), timed(step_fn(B, threads))
        result["cpu_baseline"] = {
            "value": round(B / tn, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"one sliding layer ({int(views1[0])} keys) and one global layer "
                      f"({int(views1[5])} keys) decoded, a step priced as 25 + 5 of them; f32 "
                      f"dequantize-then-attend, median of 3 after a warm-up: batch row 0 at 1 "
                      f"thread, all {B} rows at {threads} threads",
            "single_thread": {"value": round(1.0 / t1, 3), "unit": "tokens/s", "cores": 1,
                              "s_per_step": round(t1, 4)},
            "s_per_step": round(tn, 4), "cpu_model": _cpu_model(), "cpus_visible": os.cpu_count()}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
