"""Batched randomized SVD on the GPU (HIP compressor kernel).

API of unsloth_spectral/rsvd.py:28-157 (``batched_randomized_svd``).  The
kernel evaluates the reference's subspace -- Y = (M M^T)^q M Omega, Q = qr(Y),
Bp = Q^T M, svd(Bp), U = Q U~ -- re-orthonormalising after every product so
that fp32 rounding cannot wash out the small directions (Halko et al. 2011,
Alg. 4.4; the same span in exact arithmetic).  Omega is drawn on the device
(Philox4x32-10 + Box-Muller) unless given; pass the reference's draw to
reproduce its sketch.
"""
import ctypes
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check, ptr


def compress_matrices(M: torch.Tensor, k: int, n_iter: int = 2, oversampling: int = 5,
                      omega: Optional[torch.Tensor] = None, seed: int = 0, granularity: str = "per_head",
                      coeff_major: bool = False, basis_dmajor: bool = False, debug: bool = False,
                      row_weights: Optional[torch.Tensor] = None):
    """Compresses M [N, m, n] into INT8 codes + scales + fp16 basis.

    ``row_weights`` ([m] shared by every matrix, or [N, m]; positive) selects
    attention-weighted compression (spectral_cache.py:351-393): the SVD of
    diag(w) M with w = sqrt(a / mean(a)), coefficients divided by w.

    Returns a dict with ``codes`` (int8 [N, m, kp] or [N, kp, m]), ``scales``
    (f32 [N] or [N, m]), ``minmax`` [N, 2], ``vnorm`` [N], ``basis`` (f16
    [N, kp, n] or [N, n, kp]), ``kp``, ``r``; with ``debug`` also fp32
    ``coeffs`` [N, m, k], ``svals`` [N, k], ``vh`` [N, k, n], ``omega``."""
    _lib.require_device(M, "M")
    if M.dim() != 3:
        raise ValueError("M must be [batch, m, n]")
    N, m, n = M.shape
    if M.dtype not in _lib.SC_DTYPE:
        raise TypeError(f"unsupported dtype {M.dtype}")
    r = min(k + oversampling, min(m, n))
    from .spectral_cache import padded_rank
    kp = padded_rank(k)
    dev = M.device
    Mc = M
    epr = 4 if M.dtype == torch.float32 else 8
    if Mc.stride(-1) != 1 or Mc.stride(1) % epr or Mc.stride(0) % epr or Mc.data_ptr() % 16:
        Mc = Mc.contiguous()
    per_row = granularity == "per_row"
    codes = torch.empty((N, kp, m) if coeff_major else (N, m, kp), dtype=torch.int8, device=dev)
    scales = torch.empty((N, m) if per_row else (N,), dtype=torch.float32, device=dev)
    minmax = torch.empty(N, 2, dtype=torch.float32, device=dev)
    vnorm = torch.empty(N, dtype=torch.float32, device=dev)
    basis = torch.empty((N, n, kp) if basis_dmajor else (N, kp, n), dtype=torch.float16, device=dev)
    om = None
    if omega is not None:
        om = omega.to(device=dev, dtype=torch.float32).contiguous()
        if om.shape != (N, n, r):
            raise ValueError(f"omega must be [{N}, {n}, {r}], got {tuple(om.shape)}")
    dbg = {}
    if debug:
        dbg = {"coeffs": torch.empty(N, m, k, dtype=torch.float32, device=dev),
               "svals": torch.empty(N, k, dtype=torch.float32, device=dev),
               "vh": torch.empty(N, k, n, dtype=torch.float32, device=dev),
               "omega": torch.empty(N, n, r, dtype=torch.float32, device=dev)}
    a = _lib.ScCompressArgs()
    a.count, a.inner, a.rows, a.cols, a.rank = N, 1, m, n, k
    a.oversample, a.n_iter, a.kp = oversampling, n_iter, kp
    a.granularity = _lib.GRANULARITY[granularity]
    a.coeff_major, a.basis_dmajor = int(coeff_major), int(basis_dmajor)
    a.m_dtype = _lib.SC_DTYPE[M.dtype]
    a.m = Mc.data_ptr()
    a.m_stride_outer, a.m_stride_inner, a.m_stride_row = Mc.stride(0), 0, Mc.stride(1)
    a.omega = om.data_ptr() if om is not None else None
    a.seed = seed & 0xFFFFFFFFFFFFFFFF
    a.codes, a.codes_stride_outer = codes.data_ptr(), codes.stride(0)
    a.scales, a.scales_stride_outer = scales.data_ptr(), (m if per_row else 1)
    a.minmax, a.minmax_stride_outer = minmax.data_ptr(), 2
    a.vnorm, a.vnorm_stride_outer = vnorm.data_ptr(), 1
    a.basis, a.basis_stride_outer = basis.data_ptr(), basis.stride(0)
    if debug:
        a.coeffs_out = dbg["coeffs"].data_ptr()
        a.svals_out = dbg["svals"].data_ptr()
        a.vh_out = dbg["vh"].data_ptr()
        a.omega_out = dbg["omega"].data_ptr()
    rw = None
    if row_weights is not None:
        rw = row_weights.to(device=dev, dtype=torch.float32).contiguous()
        if rw.shape == (m,):
            a.row_weights_stride_outer = 0
        elif rw.shape == (N, m):
            a.row_weights_stride_outer = m
        else:
            raise ValueError(f"row_weights must be [{m}] or [{N}, {m}], got {tuple(rw.shape)}")
        a.row_weights = rw.data_ptr()
    check(_lib.load().sc_rsvd_compress(ctypes.byref(a), _lib.stream_of(Mc)))
    out = {"codes": codes, "scales": scales, "minmax": minmax, "vnorm": vnorm, "basis": basis,
           "kp": kp, "r": r}
    out.update(dbg)
    return out


def batched_randomized_svd(
    M: torch.Tensor,
    k: int,
    n_iter: int = 2,
    oversampling: int = 5,
    omega: Optional[torch.Tensor] = None,
    seed: int = 0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Truncated SVD of every matrix of M [B, m, n]: U [B, m, k], S [B, k],
    Vh [B, k, n] in M's dtype (rsvd.py:28-157).  ``omega`` [B, n, r] fixes
    the Gaussian sketch (r = min(k + oversampling, m, n))."""
    _lib.require_device(M, "M")
    B, m, n = M.shape
    r = min(k + oversampling, min(m, n))
    if r >= min(m, n) - 1:                       # rsvd.py:84-87 full-SVD edge
        U, S, Vh = torch.linalg.svd(M.float(), full_matrices=False)
        return U[:, :, :k].to(M.dtype), S[:, :k].to(M.dtype), Vh[:, :k, :].to(M.dtype)
    res = compress_matrices(M, k, n_iter, oversampling, omega, seed, debug=True)
    S = res["svals"]
    U = torch.where(S[:, None, :] > 0, res["coeffs"] / torch.clamp(S[:, None, :], min=1e-30),
                    torch.zeros_like(res["coeffs"]))
    return U.to(M.dtype), S.to(M.dtype), res["vh"].to(M.dtype)
