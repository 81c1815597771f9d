"""The oracle's cache index math against the digests the reference recorded.

The reference drives every cache kind through fixed plans (prefill chunks,
decode across the 256-token growth step and around the ring, rewinds) and
folds every fetched view, backing buffer and counter into an FNV-1a digest
(crates/lumen-mlx/src/native_cache/golden_tests.rs:413-497). The values below
are copied from those recordings. Matching them pins step-256 growth, ring
rotation, the concat/trim path, rewinds and (for the affine kinds) MLX's
4-bit gs64 quantizer, bit for bit.
"""
import pytest

from oracle_lib import golden_digest

RECORDED = [
    # (kind, plan, prealloc, digest) -- golden_tests.rs:413-497
    ("full", "full", False, 0x27B1CA76B702EBF0),
    ("full", "full", True, 0xF074133E39CC9BFF),
    ("quant_full", "full", False, 0x68F1E4FA5D294418),
    ("quant_full", "full", True, 0xE3D184F221CB6D4E),
    ("rot", "small", False, 0x5834E15BBC8D76B6),
    ("rot", "small", True, 0xD1F88E7DFD07EA48),
    ("rot", "large", False, 0x2AA678ACAFCD12FF),
    ("rot", "large", True, 0x72AA165F2E2BD6CF),
    ("rot_quant", "small", False, 0xCC42D273A7D56080),
    ("rot_quant", "small", True, 0xF3A5DD7DBE5223CE),
    ("rot_quant", "large", False, 0x7418140411240BFC),
    ("rot_quant", "large", True, 0x2812FEB187CCFF94),
    ("tq", "small", False, 0x317E3BFF116A9EE8),
    ("tq", "small", True, 0xECCE0A8165FC6B99),
    ("tq", "large", False, 0x9212159C7532A30B),
    ("tq", "large", True, 0x4F12B91EE3F90B33),
    ("tq", "full", False, 0xF9CAB87F57FB453B),
    ("tq", "full", True, 0xF2CF59207A0C8E31),
    ("tq_qjl", "small", False, 0x0F372B77B7090518),
    ("tq_qjl", "small", True, 0x602909E0D05E6F27),
    ("tq_qjl", "large", False, 0xE01557C21B1FD2CE),
    ("tq_qjl", "large", True, 0xB978336B3D4715D2),
    ("tq_qjl", "full", False, 0x2931526276ECF5F7),
    ("tq_qjl", "full", True, 0xC0A764840E88A73B),
]


@pytest.mark.parametrize("kind,plan,prealloc,want", RECORDED)
def test_digest_matches_reference_recording(kind, plan, prealloc, want):
    assert golden_digest(kind, plan, prealloc) == want


@pytest.mark.parametrize("kind,plan,prealloc,want",
                         [r for r in RECORDED if r[0] in ("quant_full", "rot_quant")])
def test_half_even_rounding_is_rejected_by_the_recording(kind, plan, prealloc, want):
    # A planted mistake: MLX's CPU fallback rounds half to even. The recording
    # was made on the Metal kernel, which rounds half away from zero, and the
    # digests tell the two apart.
    assert golden_digest(kind, plan, prealloc, round_mode=1) != want
