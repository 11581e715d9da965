"""Attention-weighted compression and landmark tokens (spectral_cache.py:
321-407, :710-852) through the HIP compressor, against the oracle.

Bars: the weighted reconstruction error within 1% relative of the float64
oracle with the same Omega and importances (measured to 2e-3), singular
values of the weighted problem to 1e-4, INT8 codes and scales bit-exact
with the oracle's quantiser on the kernel's coefficients; constant
importances (w = 1 exactly) bit-identical to the unweighted fp32 path."""
import numpy as np
import pytest
import torch

from helpers import lowrank_plus_noise
from oracle.cache import compress_tensor, row_weights
from oracle.quant import quantize_per_head
from oracle.rsvd import per_matrix_error, randomized_svd_subspace64

pytestmark = pytest.mark.gpu


def _weighted_err(M, C, B, w):
    """||diag(w)(M - C B)||_F / ||diag(w) M||_F per matrix; w [N, m]."""
    M = np.asarray(M, np.float64)
    R = np.asarray(C, np.float64) @ np.asarray(B, np.float64)
    num = np.linalg.norm((w[:, :, None] * (M - R)).reshape(M.shape[0], -1), axis=1)
    den = np.linalg.norm((w[:, :, None] * M).reshape(M.shape[0], -1), axis=1)
    return num / den


@pytest.mark.parametrize("shared", [True, False])
def test_weighted_against_oracle(shared):
    from unsloth_spectral import compress_matrices
    rng = np.random.default_rng(11 + shared)
    N, m, n, k = 8, 512, 128, 16
    M = lowrank_plus_noise(rng, N, m, n)
    omega = rng.standard_normal((N, n, k + 5)).astype(np.float32)
    imp = rng.uniform(0.05, 4.0, m if shared else (N, m)).astype(np.float32)
    imp_n = np.broadcast_to(imp, (N, m))
    res = compress_matrices(torch.from_numpy(M).cuda(), k, omega=torch.from_numpy(omega).cuda(), debug=True,
                            row_weights=torch.from_numpy(imp).cuda())
    torch.cuda.synchronize()
    C, Vh, S = res["coeffs"].cpu().numpy(), res["vh"].cpu().numpy(), res["svals"].cpu().numpy()
    W = np.stack([row_weights(imp_n[i]) for i in range(N)]).astype(np.float64)
    Mw = (M.astype(np.float32) * W[:, :, None].astype(np.float32)).astype(np.float32)
    U64, S64, V64 = randomized_svd_subspace64(Mw, k, omega)
    C64 = U64 * S64[:, None, :] / W[:, :, None]
    e_gpu = _weighted_err(M, C, Vh, W)
    e64 = _weighted_err(M, C64, V64, W)
    np.testing.assert_allclose(e_gpu, e64, rtol=2e-3)
    np.testing.assert_allclose(S, S64, rtol=1e-4)
    # unweighted error of the weighted fit agrees with the oracle's too
    np.testing.assert_allclose(per_matrix_error(M, C, Vh), per_matrix_error(M, C64, V64), rtol=1e-2)
    codes, scale, _, _ = quantize_per_head(C)
    np.testing.assert_array_equal(res["codes"][:, :, :k].cpu().numpy(), codes)
    np.testing.assert_array_equal(res["scales"].cpu().numpy(), scale)


def test_oracle_compress_tensor_weighted_matches_kernel_path():
    """oracle.cache.compress_tensor (weighted, float64 subspace) vs the
    kernel on one [H, T, D] block: reconstruction errors to 2e-3."""
    from unsloth_spectral import compress_matrices
    rng = np.random.default_rng(5)
    H, T, D, k = 4, 512, 128, 32
    X = lowrank_plus_noise(rng, H, T, D)
    omega = rng.standard_normal((H, D, k + 5)).astype(np.float32)
    imp = rng.uniform(0.1, 2.0, T).astype(np.float32)
    *_, c_or = compress_tensor(X, k, omega, algorithm="subspace64", attention_weights=imp)
    _, _, b_or, _, _ = compress_tensor(X, k, omega, algorithm="subspace64", attention_weights=imp)
    res = compress_matrices(torch.from_numpy(X).cuda(), k, omega=torch.from_numpy(omega).cuda(), debug=True,
                            row_weights=torch.from_numpy(imp).cuda())
    e_gpu = per_matrix_error(X, res["coeffs"].cpu().numpy(), res["vh"].cpu().numpy())
    e_or = per_matrix_error(X, c_or, b_or.astype(np.float32))
    np.testing.assert_allclose(e_gpu, e_or, rtol=2e-3)


def test_constant_weights_equal_unweighted_fp32_path():
    from unsloth_spectral import compress_matrices
    rng = np.random.default_rng(3)
    M = torch.from_numpy(lowrank_plus_noise(rng, 4, 256, 64).astype(np.float32)).cuda()
    omega = torch.from_numpy(rng.standard_normal((4, 64, 13)).astype(np.float32)).cuda()
    a = compress_matrices(M, 8, omega=omega, debug=True)
    b = compress_matrices(M, 8, omega=omega, debug=True, row_weights=torch.full((256,), 0.5, device="cuda"))
    for key in ("codes", "scales", "basis", "coeffs", "svals", "vh"):
        assert torch.equal(a[key], b[key]), key


def test_row_weights_shape_is_checked():
    from unsloth_spectral import compress_matrices
    M = torch.zeros(2, 128, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        compress_matrices(M, 4, row_weights=torch.ones(64, device="cuda"))


def _cache(H=2, D=128, T=128, weighted=True):
    from unsloth_spectral import SpectralCache
    return SpectralCache(H, D, block_size=T, k_rank_keys=8, k_rank_values=8, device="cuda",
                         use_attention_weighted_svd=weighted)


def test_compress_tensor_api():
    """_compress_tensor returns dequantised coefficients, the basis and
    per-head (min, max); a rank-4 block comes back within INT8 rounding,
    weighted or not; without the flag the weights are ignored."""
    rng = np.random.default_rng(7)
    H, T, D = 2, 128, 128
    X = (rng.standard_normal((1, H, T, 4)) @ rng.standard_normal((1, H, 4, D))).astype(np.float16)
    Xt = torch.from_numpy(X).cuda()
    imp = torch.from_numpy(rng.uniform(0.1, 5.0, T).astype(np.float32)).cuda()
    for weighted in (True, False):
        cache = _cache(H, D, T, weighted)
        coeffs, basis, scales = cache._compress_tensor(Xt, 8, attention_weights=imp)
        assert coeffs.shape == (H, T, 8) and basis.shape == (H, 8, D) and scales.shape == (H, 2)
        assert coeffs.dtype == torch.float16 and basis.dtype == torch.float16
        R = torch.bmm(coeffs.float(), basis.float())
        rel = ((R - Xt[0].float()).norm() / Xt.float().norm()).item()
        assert rel < 3e-2, rel   # per-head INT8 rounding of the coefficients
        assert torch.all(scales[:, 0] <= scales[:, 1])
        amax = coeffs.float().abs().amax(dim=(1, 2))
        np.testing.assert_allclose(amax.cpu().numpy(), scales.abs().amax(dim=1).cpu().numpy(), rtol=1e-2)


def test_attention_importance_running_average():
    """spectral_cache.py:710-777: first update stores the mean over
    (batch, heads, query), later ones mix with alpha = 0.1 after padding."""
    cache = _cache()
    a1 = torch.rand(1, 4, 1, 256, device="cuda")
    a2 = torch.rand(1, 4, 1, 384, device="cuda")
    cache.update_attention_importance(a1, 255)
    np.testing.assert_allclose(cache.attention_importance.cpu().numpy(), a1.mean(dim=(0, 1, 2)).cpu().numpy())
    cache.update_attention_importance(a2, 383)
    m1, m2 = a1.mean(dim=(0, 1, 2)).cpu().numpy(), a2.mean(dim=(0, 1, 2)).cpu().numpy()
    want = np.concatenate([m1, np.zeros(128, np.float32)]) * 0.9 + 0.1 * m2
    np.testing.assert_allclose(cache.attention_importance.cpu().numpy(), want, rtol=1e-6)
    assert cache.get_block_attention_weights(2).shape == (128,)
    assert cache.get_block_attention_weights(3) is None
    plain = _cache(weighted=False)
    plain.update_attention_importance(a1, 255)
    assert plain.attention_importance is None and plain.get_block_attention_weights(0) is None


def test_landmarks_come_first():
    """spectral_cache.py:779-852: landmarks, then reconstructed cold blocks,
    then the FP16 tail, with their positions."""
    rng = np.random.default_rng(9)
    H, D, T = 2, 128, 128
    cache = _cache(H, D, T, weighted=False)
    assert cache.get_kv_with_landmarks() == (None, None, None)
    LK = torch.from_numpy(rng.standard_normal((1, H, 3, D)).astype(np.float16)).cuda()
    LV = torch.from_numpy(rng.standard_normal((1, H, 3, D)).astype(np.float16)).cuda()
    cache.add_landmarks(LK[:, :, :2], LV[:, :, :2], torch.tensor([[0, 1]], device="cuda"))
    cache.add_landmarks(LK[:, :, 2:], LV[:, :, 2:], torch.tensor([[2]], device="cuda"))
    K, V, pos = cache.get_kv_with_landmarks()
    assert torch.equal(K, LK) and torch.equal(V, LV) and pos.tolist() == [[0, 1, 2]]
    A = torch.from_numpy(rng.standard_normal((1, H, T + 40, D)).astype(np.float16)).cuda()
    cache.append(A, A)
    K, V, pos = cache.get_kv_with_landmarks()
    Kc, Vc = cache.get_kv()
    assert K.shape == (1, H, 3 + T + 40, D)
    assert torch.equal(K[:, :, :3], LK) and torch.equal(V[:, :, :3], LV)
    assert torch.equal(K[:, :, 3:], Kc) and torch.equal(V[:, :, 3:], Vc)
    assert pos.tolist() == [[0, 1, 2] + list(range(T + 40))]
    cache.reset()
    assert cache.landmark_K is None and cache.get_kv_with_landmarks() == (None, None, None)


def test_landmarks_with_two_sequences():
    """Positions are per sequence ([B, T]) for every tier."""
    rng = np.random.default_rng(10)
    H, D, T = 2, 128, 128
    cache = _cache(H, D, T, weighted=False)
    A = torch.from_numpy(rng.standard_normal((2, H, T + 8, D)).astype(np.float16)).cuda()
    # the two sequences sit at different positions (sequence 1 starts at 1000)
    start = torch.tensor([[0], [1000]], device="cuda")
    cache.append(A, A, start + torch.arange(T + 8, device="cuda")[None])
    L = torch.from_numpy(rng.standard_normal((2, H, 1, D)).astype(np.float16)).cuda()
    cache.add_landmarks(L, L, torch.tensor([[0], [7]], device="cuda"))
    K, V, pos = cache.get_kv_with_landmarks()
    assert K.shape == (2, H, 1 + T + 8, D) and pos.shape == (2, 1 + T + 8)
    assert pos[:, 0].tolist() == [0, 7]
    assert pos[0, 1:].tolist() == list(range(T + 8))
    assert pos[1, 1:].tolist() == list(range(1000, 1000 + T + 8))   # cold block of sequence 1, then its tail
    assert cache.positions().tolist() == pos[:, 1:].tolist()
    Kc, _ = cache.get_kv()
    assert torch.equal(K[:, :, 1:], Kc)
