"""INT8 symmetric quantisation, restated from the reference (test infrastructure).

Reference: unsloth_spectral/spectral_cache.py
  * per-head  ``_quantize_int8_batched``  :481-516
  * per-tensor ``_quantize_int8``         :452-479
The reference only *simulates* INT8: it returns ``round(x/scale)*scale``
in float32 (later cast to the model dtype, :404) and stores ``[min, max]``
instead of the scale (:511-514).  Here the codes are returned explicitly so
that the HIP quantiser can be compared bit for bit.

Arithmetic that fixes bit-exactness (all float32):
  absmax = max(max|x|, float32(1e-8))     (:501-504)
  scale  = absmax / float32(127.0)        (:505, IEEE division)
  code   = round_half_even(x / scale)     (:508, IEEE division, torch.round)
The per-row granularity uses the same formula with one scale per row (the
layout of the benchmark workloads; it has no reference counterpart).
"""
import numpy as np

EPS = np.float32(1e-8)
Q127 = np.float32(127.0)


def _quantize(x, axes):
    x = np.asarray(x, dtype=np.float32)
    tmin = x.min(axis=axes, keepdims=True)
    tmax = x.max(axis=axes, keepdims=True)
    absmax = np.maximum(np.abs(x).max(axis=axes, keepdims=True), EPS)
    scale = (absmax / Q127).astype(np.float32)
    codes = np.rint(x / scale).astype(np.float32)
    deq = (codes * scale).astype(np.float32)
    return codes.astype(np.int8), scale, deq, tmin, tmax


def quantize_per_head(x):
    """spectral_cache.py:481-516 -- one scale per leading index ("head").

    Returns (codes int8 like x, scale [H] f32, dequantised f32 like x,
    minmax [H, 2] f32 -- the reference's ``scales`` output)."""
    x = np.asarray(x, dtype=np.float32)
    axes = tuple(range(1, x.ndim))
    codes, scale, deq, tmin, tmax = _quantize(x, axes)
    h = x.shape[0]
    minmax = np.concatenate([tmin.reshape(h, 1), tmax.reshape(h, 1)], axis=1)
    return codes, scale.reshape(h), deq, minmax


def quantize_per_row(x):
    """Per-row variant (one scale per row of the last axis)."""
    x = np.asarray(x, dtype=np.float32)
    codes, scale, deq, tmin, tmax = _quantize(x, (x.ndim - 1,))
    return codes, scale[..., 0], deq, np.stack([tmin[..., 0], tmax[..., 0]], -1)


def quantize_per_tensor(x):
    """spectral_cache.py:452-479 -- one scale for the whole tensor."""
    x = np.asarray(x, dtype=np.float32)
    codes, scale, deq, tmin, tmax = _quantize(x, tuple(range(x.ndim)))
    return codes, scale.reshape(()), deq, np.array([tmin.item(), tmax.item()], np.float32)


def codes_from_reference_block(coeffs_fp16, minmax):
    """Recover INT8 codes from a reference SpectralBlock.

    The reference stores fp16(code*scale) and [min, max] per head
    (spectral_cache.py:404, :511-514).  scale = max(|min|,|max|,1e-8)/127 and
    code = round(coeff/scale) is exact because the FP16 cast moves a
    coefficient by at most 2^-11 * 127 * scale < 0.07 * scale."""
    mm = np.asarray(minmax, np.float32)
    absmax = np.maximum(np.maximum(np.abs(mm[:, 0]), np.abs(mm[:, 1])), EPS)
    scale = (absmax / Q127).astype(np.float32)
    c = np.asarray(coeffs_fp16, np.float32)
    shape = (-1,) + (1,) * (c.ndim - 1)
    codes = np.rint(c / scale.reshape(shape)).astype(np.int8)
    return codes, scale
