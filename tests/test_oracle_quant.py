"""Pins the INT8 quantiser restatement (oracle/quant.py) with known answers.

Reference: unsloth_spectral/spectral_cache.py:452-516.  Each check fixes a
plausible mistake: ties must go to even (torch.round), the scale is
absmax/127 with the 1e-8 floor, the absmax element maps to +-127, codes are
recoverable from the reference's fp16 coefficients."""
import json
import os

import numpy as np
import pytest

from oracle.quant import codes_from_reference_block, quantize_per_head, quantize_per_row, quantize_per_tensor

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_ties_go_to_even_known_answers():
    # absmax = 127/16 -> scale = 1/16 exactly; x/scale has exact .5 ties.
    s = np.float32(1 / 16)
    halves = np.array([127.0, 0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5, 126.5, -126.5], np.float32)
    x = (halves * s)[None, None, :]
    codes, scale, deq, minmax = quantize_per_head(x)
    assert scale[0] == s
    assert codes[0, 0].tolist() == [127, 0, 2, 2, 4, 0, -2, -2, -4, 126, -126]
    assert minmax.tolist() == [[float(x.min()), float(x.max())]]
    np.testing.assert_array_equal(deq, codes.astype(np.float32) * s)


def test_all_zero_uses_floor_scale():
    codes, scale, deq, _ = quantize_per_head(np.zeros((2, 5, 3), np.float32))
    assert np.all(codes == 0)
    assert np.all(scale == np.float32(np.float32(1e-8) / np.float32(127.0)))


def test_absmax_maps_to_127_and_sign_symmetry():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, 64, 16)).astype(np.float32)
    c1, s1, _, _ = quantize_per_head(x)
    c2, s2, _, _ = quantize_per_head(-x)
    np.testing.assert_array_equal(c1, -c2)
    np.testing.assert_array_equal(s1, s2)
    for h in range(4):
        i = np.unravel_index(np.abs(x[h]).argmax(), x[h].shape)
        assert abs(int(c1[h][i])) == 127
    assert np.abs(c1).max() == 127


def test_per_row_and_per_tensor_scales():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 8, 16)).astype(np.float32)
    x[1, 3] *= 10
    c, s, _, _ = quantize_per_row(x)
    assert s.shape == (2, 8)
    np.testing.assert_array_equal(s, np.maximum(np.abs(x).max(-1), np.float32(1e-8)) / np.float32(127))
    assert np.all(np.abs(c).max(-1) == 127)
    ct, st, _, mm = quantize_per_tensor(x)
    assert st == np.abs(x).max() / np.float32(127)
    assert mm.tolist() == [float(x.min()), float(x.max())]


def test_codes_recovered_from_reference_fp16_coefficients():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((8, 512, 32)) * 3).astype(np.float32)
    codes, scale, deq, minmax = quantize_per_head(x)
    ref_coeffs = deq.astype(np.float16)          # what the reference stores (:404)
    rec, rscale = codes_from_reference_block(ref_coeffs, minmax)
    np.testing.assert_array_equal(rscale, scale)
    np.testing.assert_array_equal(rec, codes)


def test_golden_quant_vectors():
    path = os.path.join(GOLDEN, "quant_vectors.npz")
    if not os.path.exists(path):
        pytest.skip("fixture missing (run tests/golden/make_golden.py)")
    g = np.load(path)
    c, s, _, _ = quantize_per_head(g["x"])
    np.testing.assert_array_equal(c, g["codes_per_head"])
    np.testing.assert_array_equal(s, g["scales_per_head"])
    c, s, _, _ = quantize_per_row(g["x"])
    np.testing.assert_array_equal(c, g["codes_per_row"])
    np.testing.assert_array_equal(s, g["scales_per_row"])
