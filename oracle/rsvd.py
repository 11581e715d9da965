"""Batched randomized SVD, restated from the reference (test infrastructure).

Reference: unsloth_spectral/rsvd.py:28-157 (``batched_randomized_svd``),
self-test :160-220.  Called with k = rank, n_iter = 2, oversampling = 5 from
unsloth_spectral/spectral_cache.py:374 on ``X.squeeze(0).float()`` (:349).

Two functions:

* ``randomized_svd_ref`` -- the reference's op order in float32 with LAPACK
  (numpy.linalg): Y = M Omega, n_iter x Y = M (M^T Y) with no
  re-orthonormalisation, Q = qr(Y), Bp = Q^T M, svd(Bp), U = Q U~,
  truncate to k.  Includes the full-SVD edge case r >= min(m, n) - 1
  (rsvd.py:84-87).
* ``randomized_svd_subspace64`` -- the same subspace in exact arithmetic,
  evaluated stably in float64: every power-iteration product is
  re-orthonormalised (Halko et al. 2011, Alg. 4.4).  span(Q) equals the
  reference's span(Y) in exact arithmetic, so U S Vh agree up to the signs
  of singular vectors; this is the algorithm the HIP kernel evaluates and
  the tight comparison target for it.
"""
import numpy as np


def oversampled_rank(k, m, n, oversampling=5):
    """rsvd.py:75"""
    return min(k + oversampling, min(m, n))


def randomized_svd_ref(M, k, omega, n_iter=2, oversampling=5):
    """rsvd.py:74-157 in float32.  ``omega`` is the [B, n, r] Gaussian draw of
    rsvd.py:95 (the first RNG draw of the call)."""
    M = np.asarray(M, dtype=np.float32)
    b, m, n = M.shape
    r = oversampled_rank(k, m, n, oversampling)
    if r >= min(m, n) - 1:                                   # rsvd.py:84-87
        U, S, Vh = np.linalg.svd(M, full_matrices=False)
        return U[:, :, :k], S[:, :k], Vh[:, :k, :]
    omega = np.asarray(omega, dtype=np.float32)
    assert omega.shape == (b, n, r), (omega.shape, (b, n, r))
    Y = np.matmul(M, omega)                                  # :100
    Mt = np.ascontiguousarray(M.transpose(0, 2, 1))
    for _ in range(n_iter):                                  # :111-113
        Y = np.matmul(M, np.matmul(Mt, Y))
    Q, _ = np.linalg.qr(Y)                                   # :122
    Bp = np.matmul(Q.transpose(0, 2, 1), M)                  # :132
    Ut, S, Vh = np.linalg.svd(Bp, full_matrices=False)       # :141
    U = np.matmul(Q, Ut)                                     # :149
    return U[:, :, :k], S[:, :k], Vh[:, :k, :]               # :157


def _orth(A):
    q, _ = np.linalg.qr(A)
    return q


def randomized_svd_subspace64(M, k, omega, n_iter=2, oversampling=5):
    """Same subspace as ``randomized_svd_ref``, evaluated in float64 with
    re-orthonormalisation after every product."""
    M = np.asarray(M, dtype=np.float64)
    b, m, n = M.shape
    r = oversampled_rank(k, m, n, oversampling)
    if r >= min(m, n) - 1:
        U, S, Vh = np.linalg.svd(M, full_matrices=False)
        return U[:, :, :k], S[:, :k], Vh[:, :k, :]
    Mt = M.transpose(0, 2, 1)
    Q = _orth(np.matmul(M, np.asarray(omega, np.float64)))
    for _ in range(n_iter):
        Z = _orth(np.matmul(Mt, Q))
        Q = _orth(np.matmul(M, Z))
    Bp = np.matmul(Q.transpose(0, 2, 1), M)
    Ut, S, Vh = np.linalg.svd(Bp, full_matrices=False)
    U = np.matmul(Q, Ut)
    return U[:, :, :k], S[:, :k], Vh[:, :k, :]


def reconstruction_error(M, U, S, Vh):
    """||M - U diag(S) Vh||_F / ||M||_F over the whole batch (rsvd.py:189-193)."""
    M = np.asarray(M, np.float64)
    R = np.matmul(np.asarray(U, np.float64) * np.asarray(S, np.float64)[:, None, :],
                  np.asarray(Vh, np.float64))
    return float(np.linalg.norm(M - R) / np.linalg.norm(M))


def per_matrix_error(M, C, Bas):
    """||M_i - C_i B_i||_F / ||M_i||_F for every matrix of the batch."""
    M = np.asarray(M, np.float64)
    R = np.matmul(np.asarray(C, np.float64), np.asarray(Bas, np.float64))
    num = np.linalg.norm((M - R).reshape(M.shape[0], -1), axis=1)
    den = np.linalg.norm(M.reshape(M.shape[0], -1), axis=1)
    return num / np.maximum(den, 1e-300)
