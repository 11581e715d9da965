"""INT8 quantiser: HIP kernel bit-exact against the oracle (codes and scales)
when fed the same float32 coefficients."""
import os

import numpy as np
import pytest
import torch

from oracle.quant import quantize_per_head, quantize_per_row, quantize_per_tensor

pytestmark = pytest.mark.gpu


def _gpu_quant(x, gran):
    import ctypes
    from unsloth_spectral import _lib
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    G, R, C = x.shape
    codes = torch.empty(x.shape, dtype=torch.int8, device="cuda")
    ns = {0: G, 1: G * R, 2: 1}[gran]
    scales = torch.empty(ns, dtype=torch.float32, device="cuda")
    mm = torch.empty(G * 2 if gran != 2 else 2, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load().sc_quantize_int8(ctypes.c_void_p(xt.data_ptr()), G, R, C, gran,
                                            ctypes.c_void_p(codes.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
                                            ctypes.c_void_p(mm.data_ptr()), None))
    torch.cuda.synchronize()
    return codes.cpu().numpy(), scales.cpu().numpy(), mm.cpu().numpy()


@pytest.mark.parametrize("shape", [(8, 512, 16), (8, 512, 32), (3, 7, 5), (1, 1, 1)])
def test_per_head_bit_exact(shape):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(shape) * rng.uniform(0.01, 30, size=(shape[0], 1, 1))).astype(np.float32)
    c, s, mm = _gpu_quant(x, 0)
    rc, rs, _, rmm = quantize_per_head(x)
    np.testing.assert_array_equal(c, rc)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(mm.reshape(-1, 2), rmm)


@pytest.mark.parametrize("shape", [(8, 512, 32), (2, 3, 100)])
def test_per_row_bit_exact(shape):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(shape) * 4).astype(np.float32)
    x[0, 1] = 0.0
    c, s, mm = _gpu_quant(x, 1)
    rc, rs, _, _ = quantize_per_row(x)
    np.testing.assert_array_equal(c, rc)
    np.testing.assert_array_equal(s.reshape(rs.shape), rs)


def test_per_tensor_bit_exact():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 64, 8)).astype(np.float32)
    c, s, mm = _gpu_quant(x, 2)
    rc, rs, _, rmm = quantize_per_tensor(x)
    np.testing.assert_array_equal(c, rc)
    assert s[0] == rs
    np.testing.assert_array_equal(mm, rmm)


def test_golden_ties_and_zeros():
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_vectors.npz"))
    c, s, _ = _gpu_quant(g["x"], 0)
    np.testing.assert_array_equal(c, g["codes_per_head"])
    np.testing.assert_array_equal(s, g["scales_per_head"])
    c, s, _ = _gpu_quant(g["x"], 1)
    np.testing.assert_array_equal(c, g["codes_per_row"])
    np.testing.assert_array_equal(s.reshape(g["scales_per_row"].shape), g["scales_per_row"])
