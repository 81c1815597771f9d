"""Shared inputs of the page-sparse tests: the reference's planted-page
scenario (native_attention.rs:1085-1140) and a checker for a page choice
against the oracle's bounds."""
import numpy as np

import oracle_lib as O
from inputs import kv_bf16

PAGE = 64


def cosine(a, b):
    a, b = a.astype(np.float64).ravel(), b.astype(np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def planted(h=8, h_kv=2, d=256, n=20_000 + 37, target_page=40):
    """Background keys N(0, 0.2^2); page `target_page` holds 4 x the mean of
    the KV head's query group, so it carries most of the attention; values
    N(0, 1). (The reference uses 16 query heads over 2 KV heads; 8 over 2
    keeps D=256 within the matrix-core layouts, H / H_kv * D / 64 <= 16.)"""
    q = kv_bf16((1, h, 1, d), 1)
    keys = O.bf16_to_f32(kv_bf16((1, h_kv, n, d), 2, std=0.2)).copy()
    qf = O.bf16_to_f32(q).reshape(1, h_kv, h // h_kv, d)
    q_kv = O.bf16_to_f32(O.bf16_from_f32(qf.mean(axis=2, keepdims=True)))
    strong = O.bf16_to_f32(O.bf16_from_f32(q_kv * np.float32(4.0)))
    keys[:, :, target_page * PAGE:(target_page + 1) * PAGE] = strong
    values = kv_bf16((1, h_kv, n, d), 3)
    return q, O.bf16_from_f32(keys), values


def check_choice(chosen, bounds, keep, tol_rel=1e-4):
    """chosen [B, H_kv, keep] must be ascending, unique, hold page 0 and the
    last four pages, and be a top-keep of the (pinned) bounds within tol."""
    B, Hkv, pages = bounds.shape
    assert chosen.shape == (B, Hkv, keep)
    for b in range(B):
        for h in range(Hkv):
            c = chosen[b, h]
            assert np.all(np.diff(c) > 0) and c[0] >= 0 and c[-1] < pages
            pinned = {0, *range(pages - 4, pages)}
            assert pinned <= set(c.tolist())
            bd = bounds[b, h].copy()
            bd[list(pinned)] = np.inf
            thr = np.sort(bd)[::-1][keep - 1]
            tol = tol_rel * (1.0 + abs(thr)) if np.isfinite(thr) else 0.0
            mask = np.zeros(pages, bool)
            mask[c] = True
            assert np.all(bd[mask] >= thr - tol), (b, h)
            assert np.all(bd[~mask] <= thr + tol), (b, h)
