"""Pins of the CPU oracle's Q4_K functions (or_q4k_half, or_q4k_dequant_block,
or_quant_q8, or_gemv_q4k), the checker of the gfx950 Q4_K GEMV.

* dequantisation: bit-exact against the reference's own dequant_block and
  half_to_float (include/nova/quant/q4_k.h, compiled unchanged into
  oracle/_ref), through the committed fixture tests/golden/q4k.npz -- which
  holds the known-answer block of tests/selftest_q4k.cpp:31-38 -- and live when
  oracle/_ref is built;
* activation quantisation (quant_kernel, src/kernel/q4k_gemv.cu:9-33): closed
  forms -- the largest |x| of each 32-block maps to +-127, d = amax/127,
  reconstruction within d/2, the 16-element sums are the sums of the codes,
  an all-zero block gives zero codes and d = 0;
* GEMV: weights whose dequantised values are known by construction (d = 1,
  dmin = 0, scales 1: every weight is its nibble) give a closed-form product,
  and the oracle equals the dot product of the dequantised rows with the
  dequantised activations.
"""
from pathlib import Path

import numpy as np
import pytest

GOLD = np.load(Path(__file__).parent / "golden" / "q4k.npz")


def test_dequant_matches_reference_fixture(oracle):
    for b, y in zip(GOLD["blocks"], GOLD["y"]):
        assert np.array_equal(oracle.q4k_dequant_block(b), y)
    for h, v in zip(GOLD["halves"], GOLD["half_values"]):
        assert oracle.q4k_half(int(h)) == v


def test_selftest_block_is_the_reference_known_answer():
    b = GOLD["blocks"][0]
    assert b[:4].view(np.uint16).tolist() == [0x2C00, 0x1A00]       # selftest_q4k.cpp:33-34


def test_dequant_live_against_reference(oracle, reference):
    if reference is None or reference.q4k is None:
        pytest.skip("oracle/_ref not built (no reference tree)")
    rng = np.random.default_rng(7)
    for _ in range(200):
        b = rng.integers(0, 256, 144, dtype=np.uint8)
        b[:4] = rng.uniform(-0.05, 0.05, 2).astype(np.float16).view(np.uint8)
        y = np.empty(256, np.float32)
        reference.q4k.ref_q4k_dequant_block(np.ascontiguousarray(b).ctypes.data, y.ctypes.data)
        assert np.array_equal(oracle.q4k_dequant_block(b), y)


def test_quant_closed_forms(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 256)).astype(np.float32) * rng.uniform(0.1, 10, (3, 1)).astype(np.float32)
    x[1, 32:64] = 0.0
    qs, d, s = oracle.quant_q8(x)
    xb = x.reshape(3, 8, 32)
    qb = qs.reshape(3, 8, 32).astype(np.int32)
    amax = np.abs(xb).max(axis=2)
    assert np.array_equal(d, (amax * np.float32(1.0 / 127.0)).astype(np.float32))
    for r in range(3):
        for b in range(8):
            if amax[r, b] == 0:
                assert not qb[r, b].any() and d[r, b] == 0
                continue
            k = np.argmax(np.abs(xb[r, b]))
            assert qb[r, b, k] == (127 if xb[r, b, k] > 0 else -127)
            assert np.abs(qb[r, b]).max() <= 127
            assert np.all(np.abs(qb[r, b] * d[r, b] - xb[r, b]) <= d[r, b] * 0.5 + 1e-6 * amax[r, b])
    assert np.array_equal(s, qs.reshape(3, 16, 16).astype(np.int32).sum(axis=2))


def test_gemv_closed_form(oracle):
    """d = 1, dmin = 0, all 6-bit scales 1: every weight equals its nibble."""
    rows, cols = 5, 512
    rng = np.random.default_rng(9)
    nib = rng.integers(0, 16, (rows, cols // 256, 256))
    blocks = np.zeros((rows, cols // 256, 144), np.uint8)
    blocks[..., 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)      # d = 1.0
    blocks[..., 4:8] = 1                                                   # scales of sub-blocks 0..3
    blocks[..., 12:16] = 1                                                 # sub-blocks 4..7 (low 4 bits)
    for g in range(4):
        lo = nib[..., 64 * g:64 * g + 32]
        hi = nib[..., 64 * g + 32:64 * g + 64]
        blocks[..., 16 + 32 * g:16 + 32 * g + 32] = (lo | (hi << 4)).astype(np.uint8)
    for r in range(rows):
        for b in range(cols // 256):
            assert np.array_equal(oracle.q4k_dequant_block(blocks[r, b]), nib[r, b].astype(np.float32))
    x = rng.standard_normal((1, cols)).astype(np.float32)
    qs, d, s = oracle.quant_q8(x)
    xq = qs[0].astype(np.float64) * np.repeat(d[0].astype(np.float64), 32)
    want = nib.reshape(rows, cols).astype(np.float64) @ xq
    got = oracle.gemv_q4k(blocks, rows, cols, qs, d, s)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
