"""Pins the rSVD restatement (oracle/rsvd.py).

* The reference's seeded self-test (rsvd.py:160-220: seed 42, B=8, m=512,
  n=128, k=16, M = randn@randn + 0.1 randn, Omega = the call's first randn)
  has a published known answer: reconstruction error 0.022725 and mean
  singular-value error 0.000072 (PHASE2_RSVD_OPTIMIZATION.md:40-41).  torch's
  CPU generator reproduces M and Omega bit for bit.
* Q^T Q = I, the Eckart-Young bound, exactness for rank <= k inputs, and the
  float64 subspace-iteration variant agreeing with the float32 restatement.
"""
import json
import os

import numpy as np
import pytest

from oracle.rsvd import (per_matrix_error, randomized_svd_ref, randomized_svd_subspace64,
                         reconstruction_error)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _seeded_case():
    torch = pytest.importorskip("torch")
    torch.manual_seed(42)
    B, m, n, k = 8, 512, 128, 16
    M = torch.randn(B, m, k) @ torch.randn(B, k, n) + 0.1 * torch.randn(B, m, n)
    omega = torch.randn(B, n, k + 5)
    return M.numpy(), omega.numpy(), k


def test_published_known_answer():
    with open(os.path.join(GOLDEN, "rsvd_known_answer.json")) as f:
        ka = json.load(f)
    M, omega, k = _seeded_case()
    assert abs(float(M.astype(np.float64).sum()) - ka["m_checksum"]) < 1e-3 * abs(ka["m_checksum"]) + 1e-3
    U, S, Vh = randomized_svd_ref(M, k, omega)
    err = reconstruction_error(M, U, S, Vh)
    assert abs(err - ka["err_published"]) < 5e-7, err
    S_full = np.linalg.svd(M.astype(np.float64), compute_uv=False)[:, :k]
    s_err = float(np.abs(S_full - S).mean())
    assert s_err < 2 * ka["s_abs_err_published"], s_err
    # rsvd.py:211-212 pass criteria
    Uf, Sf, Vf = np.linalg.svd(M.astype(np.float64), full_matrices=False)
    err_std = reconstruction_error(M, Uf[:, :, :k], Sf[:, :k], Vf[:, :k])
    assert err / err_std < 1.05
    assert float((np.abs(S_full - S) / (S_full + 1e-8)).mean()) < 0.01


def test_q_orthonormal_and_eckart_young():
    rng = np.random.default_rng(3)
    M = (rng.standard_normal((4, 256, 64)) * np.exp(-np.arange(64) / 6)).astype(np.float32)
    k = 8
    omega = rng.standard_normal((4, 64, k + 5)).astype(np.float32)
    U, S, Vh = randomized_svd_ref(M, k, omega)
    for b in range(4):
        np.testing.assert_allclose(U[b].T @ U[b], np.eye(k), atol=2e-5)
        np.testing.assert_allclose(Vh[b] @ Vh[b].T, np.eye(k), atol=2e-5)
    errs = per_matrix_error(M, U * S[:, None, :], Vh)
    Uf, Sf, Vf = np.linalg.svd(M.astype(np.float64), full_matrices=False)
    best = per_matrix_error(M, Uf[:, :, :k] * Sf[:, None, :k], Vf[:, :k])
    assert np.all(errs >= best * (1 - 1e-6))
    assert np.all(errs <= best * 1.05)


def test_exact_on_rank_deficient_inputs():
    rng = np.random.default_rng(4)
    A = rng.standard_normal((3, 128, 6)) @ rng.standard_normal((3, 6, 64))
    M = A.astype(np.float32)
    omega = rng.standard_normal((3, 64, 13)).astype(np.float32)
    U, S, Vh = randomized_svd_ref(M, 8, omega)
    assert reconstruction_error(M, U, S, Vh) < 1e-5
    U2, S2, V2 = randomized_svd_subspace64(M, 8, omega)
    assert reconstruction_error(M, U2, S2, V2) < 1e-7   # fp32 rounding of M


def test_subspace64_matches_reference_on_well_conditioned_case():
    M, omega, k = _seeded_case()
    U, S, Vh = randomized_svd_ref(M, k, omega)
    U2, S2, V2 = randomized_svd_subspace64(M, k, omega)
    np.testing.assert_allclose(S2, S, rtol=1e-5)
    e1 = per_matrix_error(M, U * S[:, None, :], Vh)
    e2 = per_matrix_error(M, U2 * S2[:, None, :], V2)
    np.testing.assert_allclose(e2, e1, rtol=1e-4)


def test_full_svd_edge_case():
    rng = np.random.default_rng(5)
    M = rng.standard_normal((2, 64, 32)).astype(np.float32)
    U, S, Vh = randomized_svd_ref(M, 28, None)     # r = 32 >= 31: full SVD branch
    assert U.shape == (2, 64, 28) and S.shape == (2, 28) and Vh.shape == (2, 28, 32)
