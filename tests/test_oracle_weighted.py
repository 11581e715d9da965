"""Pins the attention-weighted branch of the compression restatement
(oracle/cache.py: ``row_weights``, ``compress_tensor(attention_weights=)``,
restating spectral_cache.py:351-368 and :389-393).

* Known answers of the weight normalisation w = sqrt(a / mean(a)).
* Constant importances give w = 1 exactly, so the weighted branch equals the
  unweighted one bit for bit.
* A block of rank <= k is reconstructed exactly whatever the weights (a
  dropped or doubled unweighting of the coefficients fails this).
* Weighted optimality: the weighted residual ||diag(w)(X - C B)||_F is within
  5% of the optimum of the weighted problem (exact SVD of diag(w) X,
  Eckart-Young), and below the weighted residual of the unweighted fit.
"""
import numpy as np

from oracle.cache import compress_tensor, row_weights


def test_row_weight_known_answers():
    np.testing.assert_array_equal(row_weights([2.0, 2.0, 2.0, 2.0]), np.ones(4, np.float32))
    # mean 2.5 -> (0.4, 1.6) -> sqrt
    np.testing.assert_allclose(row_weights([1.0, 4.0]), [np.sqrt(0.4), np.sqrt(1.6)], rtol=1e-7)
    # mean 1/4 -> (0, 4, 0, 0) -> (0, 2, 0, 0)
    np.testing.assert_array_equal(row_weights([0.0, 1.0, 0.0, 0.0]), [0.0, 2.0, 0.0, 0.0])


def _decaying(rng, H, T, D):
    U = np.linalg.qr(rng.standard_normal((H, T, D)))[0]
    V = np.linalg.qr(rng.standard_normal((H, D, D)))[0]
    s = np.exp(-np.arange(D) / 6.0)
    return ((U * s) @ V.transpose(0, 2, 1) * 8.0 + 0.01 * rng.standard_normal((H, T, D))).astype(np.float32)


def test_constant_weights_equal_unweighted():
    rng = np.random.default_rng(0)
    X = _decaying(rng, 2, 256, 64)
    omega = rng.standard_normal((2, 64, 13)).astype(np.float32)
    a = compress_tensor(X, 8, omega)
    b = compress_tensor(X, 8, omega, attention_weights=np.full(256, 0.25, np.float32))
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_exact_for_low_rank_blocks_with_weights():
    rng = np.random.default_rng(1)
    H, T, D, r = 2, 256, 64, 5
    X = (rng.standard_normal((H, T, r)) @ rng.standard_normal((H, r, D))).astype(np.float32)
    imp = rng.uniform(0.05, 3.0, T).astype(np.float32)
    omega = rng.standard_normal((H, D, 13)).astype(np.float32)
    *_, coeffs = compress_tensor(X, 8, omega, algorithm="subspace64", attention_weights=imp)
    _, _, basis, _, _ = compress_tensor(X, 8, omega, algorithm="subspace64", attention_weights=imp)
    # reconstruct with the unquantised coefficients and the fp16 basis
    R = coeffs.astype(np.float64) @ basis.astype(np.float64)
    rel = np.linalg.norm(R - X) / np.linalg.norm(X)
    assert rel < 2e-3, rel


def test_weighted_fit_is_optimal_for_the_weighted_norm():
    rng = np.random.default_rng(2)
    H, T, D, k = 2, 256, 64, 8
    X = _decaying(rng, H, T, D)
    imp = np.where(np.arange(T) % 16 == 0, 40.0, 0.2).astype(np.float32)   # a few heavy rows
    omega = rng.standard_normal((H, D, k + 5)).astype(np.float32)
    w = row_weights(imp).astype(np.float64)

    def wres(coeffs, basis):
        R = coeffs.astype(np.float64) @ basis.astype(np.float32).astype(np.float64)
        return np.linalg.norm(w[None, :, None] * (X - R), axis=(1, 2))

    *_, cw = compress_tensor(X, k, omega, algorithm="subspace64", attention_weights=imp)
    _, _, bw, _, _ = compress_tensor(X, k, omega, algorithm="subspace64", attention_weights=imp)
    *_, cu = compress_tensor(X, k, omega, algorithm="subspace64")
    _, _, bu, _, _ = compress_tensor(X, k, omega, algorithm="subspace64")
    s = np.linalg.svd(w[None, :, None] * X.astype(np.float64), compute_uv=False)
    opt = np.sqrt((s[:, k:] ** 2).sum(axis=1))
    ew, eu = wres(cw, bw), wres(cu, bu)
    assert np.all(ew <= 1.05 * opt), (ew, opt)
    assert np.all(ew < eu), (ew, eu)
