"""The decode kernels' code-extraction plans (lumen-rs_amd/csrc/pair_plans.hpp,
written by gen_pair_plans.py), replayed on the CPU over random packed codes:
every K operand's 32-bit window ANDed with its mask must hold exactly its
codes shifted to their offsets (low and high f16 half), every V window of a
token pair exactly its channel's two codes, each code must be read exactly
once, and each must sit inside the f16 mantissa (offset + bits <= 10), which
is what makes the half the exact subnormal code * 2^(offset - 24). The
committed header must equal the generator's output."""
import os
import sys

import numpy as np
import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lumen-rs_amd",
                    "csrc")
sys.path.insert(0, CSRC)
import gen_pair_plans as G  # noqa: E402


def pack(codes, bits):
    """LSB-first u32 stream (offload/lowbit.rs:220-240)."""
    v = 0
    for i, c in enumerate(codes):
        v |= int(c) << (bits * i)
    n = len(codes) * bits // 32
    return [(v >> (32 * k)) & 0xFFFFFFFF for k in range(n)]


def window(words, bit):
    v = 0
    for k, w in enumerate(words):
        v |= w << (32 * k)
    return (v >> bit) & 0xFFFFFFFF


@pytest.mark.parametrize("bits,epl", [(b, e) for b in G.WIDTHS for e in G.EPLS[b]])
def test_plans_recover_every_code_once(bits, epl):
    rng = np.random.default_rng(bits * 100 + epl)
    top = (1 << bits) - 1
    for trial in range(4):
        c0 = rng.integers(0, top + 1, epl) if trial else np.full(epl, top)
        c1 = rng.integers(0, top + 1, epl)
        w0, w1 = pack(c0, bits), pack(c1, bits)
        seen = []
        for bit, lo, hi in G.k_plan(bits, epl):
            m = G.mask_of(lo, hi, bits)
            x = window(w0, bit) & m
            e, o = lo
            assert o + bits <= 10
            assert x & 0xFFFF == int(c0[e]) << o
            seen.append(e)
            if hi is None:
                assert x >> 16 == 0
            else:
                e2, o2 = hi
                assert o2 + bits <= 10
                assert x >> 16 == int(c0[e2]) << o2
                seen.append(e2)
        assert sorted(seen) == list(range(epl))
        seen = []
        for bit, codes in G.v_plan(bits, epl):
            merged = (window(w0, bit) & 0xFFFF) | ((window(w1, bit) & 0xFFFF) << 16)
            for e, o in codes:
                assert o + bits <= 10
                m = ((1 << bits) - 1) << o
                x = merged & (m | (m << 16))
                assert x == (int(c0[e]) << o) | ((int(c1[e]) << o) << 16)
                seen.append(e)
        assert sorted(seen) == list(range(epl))


def test_header_matches_generator(tmp_path):
    import io
    buf = io.StringIO()
    G.main(buf)
    with open(os.path.join(CSRC, "pair_plans.hpp")) as f:
        assert f.read() == buf.getvalue()
