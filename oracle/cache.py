"""Tier manager of the SpectralCache, restated from the reference (test infrastructure).

Reference: unsloth_spectral/spectral_cache.py
  * ``append``               :164-241  (new-generation reset :176-189,
                                        auto positions :199-213,
                                        concat :215-229, trigger :237-241)
  * ``_compress_hot_cache``  :243-319  (while loop over full blocks,
                                        start_position = hot_position_ids[0,0])
  * ``_compress_tensor``     :321-407  (rSVD k, n_iter=2, p=5 -> coeffs=U*S ->
                                        quantise -> fp16 casts; attention-
                                        weighted branch :351-368, :389-393)
  * ``get_spectral_components`` / ``get_all_positions`` / ``get_kv`` :518-612
One sequence (the reference asserts batch 1, :346).  ``omega_fn(kind,
block_index, shape)`` supplies the Gaussian sketch that the reference draws
with ``torch.randn`` at rsvd.py:95 (K first, then V: :285-286).
"""
import numpy as np

from .attention import ColdBlock, TierState
from .quant import quantize_per_head, quantize_per_row
from .rsvd import oversampled_rank, randomized_svd_ref, randomized_svd_subspace64


def row_weights(attention_weights):
    """spectral_cache.py:356-358: w = sqrt(a / mean(a)) in float32."""
    a = np.asarray(attention_weights, np.float32).reshape(-1)
    return np.sqrt(a / np.float32(a.mean(dtype=np.float32))).astype(np.float32)


def compress_tensor(X, rank, omega, granularity="per_head", n_iter=2, oversampling=5,
                    algorithm="reference", attention_weights=None):
    """spectral_cache.py:321-407 for X [H, T, D] (any float dtype).

    ``attention_weights`` [T] selects the attention-weighted branch
    (:351-368, :389-393): the SVD runs on X * w (w per token row) and the
    coefficients are divided by w before quantisation.

    Returns (codes int8 [H,T,k], scale f32 [H] or [H,T], basis f16 [H,k,D],
    minmax f32 [H,2], coeffs f32 [H,T,k] before quantisation)."""
    Xf = np.asarray(X, np.float32)                      # .float(), :349
    w = None
    if attention_weights is not None:
        w = row_weights(attention_weights)
        Xf = (Xf * w[None, :, None]).astype(np.float32)  # :361-362
    if algorithm == "reference":
        U, S, Vh = randomized_svd_ref(Xf, rank, omega, n_iter, oversampling)
    else:
        U, S, Vh = randomized_svd_subspace64(Xf, rank, omega, n_iter, oversampling)
    coeffs = (np.asarray(U, np.float32) * np.asarray(S, np.float32)[:, None, :]).astype(np.float32)  # :387
    if w is not None:
        coeffs = (coeffs / w[None, :, None]).astype(np.float32)          # :391-393
    if granularity == "per_head":
        codes, scale, _, minmax = quantize_per_head(coeffs)            # :398
    else:
        codes, scale, _, _ = quantize_per_row(coeffs)
        minmax = np.stack([coeffs.min(axis=(1, 2)), coeffs.max(axis=(1, 2))], -1)
    basis = np.asarray(Vh, np.float32).astype(np.float16)              # :405
    return codes, scale, basis, minmax.astype(np.float32), coeffs


class TierManager:
    """The reference SpectralCache for one sequence, with explicit codes."""

    def __init__(self, num_heads, head_dim, block_size=512, k_rank_keys=16,
                 k_rank_values=32, omega_fn=None, granularity="per_head",
                 algorithm="reference"):
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.k_rank_keys = k_rank_keys
        self.k_rank_values = k_rank_values
        self.omega_fn = omega_fn
        self.granularity = granularity
        self.algorithm = algorithm
        self.reset()

    def reset(self):
        """spectral_cache.py:137-162"""
        self.hot_K = None
        self.hot_V = None
        self.hot_pos = None
        self.blocks = []
        self.current_position = 0
        self.total_tokens = 0
        self.compression_count = 0

    def append(self, K_new, V_new, position_ids=None):
        """K_new, V_new: [H, T_new, D] (pre-RoPE); position_ids: [T_new] or None."""
        if position_ids is not None and self.total_tokens > 0:
            first = int(np.asarray(position_ids).reshape(-1)[0])
            if first < self.current_position:                  # :183
                self.reset()
        t_new = K_new.shape[1]
        if position_ids is None:
            pos = np.arange(self.current_position, self.current_position + t_new)
        else:
            pos = np.asarray(position_ids).reshape(-1).astype(np.int64)
        if self.hot_K is None:
            self.hot_K, self.hot_V, self.hot_pos = np.asarray(K_new), np.asarray(V_new), pos
        else:
            self.hot_K = np.concatenate([self.hot_K, K_new], axis=1)
            self.hot_V = np.concatenate([self.hot_V, V_new], axis=1)
            self.hot_pos = np.concatenate([self.hot_pos, pos])
        self.total_tokens += t_new
        self.current_position += t_new
        if self.hot_K.shape[1] >= self.block_size:            # :238
            self._compress_hot_cache()

    def _compress_hot_cache(self):
        while self.hot_K is not None and self.hot_K.shape[1] >= self.block_size:
            bs = self.block_size
            Kb, Vb = self.hot_K[:, :bs], self.hot_V[:, :bs]
            start = int(self.hot_pos[0])                          # :274
            idx = len(self.blocks)
            H, _, D = Kb.shape
            rk = oversampled_rank(self.k_rank_keys, bs, D)
            rv = oversampled_rank(self.k_rank_values, bs, D)
            om_k = self.omega_fn("K", idx, (H, D, rk))
            om_v = self.omega_fn("V", idx, (H, D, rv))
            ck, sk, bk, _, _ = compress_tensor(Kb, self.k_rank_keys, om_k, self.granularity,
                                               algorithm=self.algorithm)
            cv, sv, bv, _, _ = compress_tensor(Vb, self.k_rank_values, om_v, self.granularity,
                                               algorithm=self.algorithm)
            self.blocks.append(ColdBlock(ck, sk, bk, cv, sv, bv, start))
            self.compression_count += 1
            if self.hot_K.shape[1] > bs:                          # :304-308
                self.hot_K, self.hot_V = self.hot_K[:, bs:], self.hot_V[:, bs:]
                self.hot_pos = self.hot_pos[bs:]
            else:
                self.hot_K = self.hot_V = self.hot_pos = None
                break

    def state(self):
        return TierState(list(self.blocks), self.hot_K, self.hot_V, self.hot_pos)

    def get_all_positions(self):
        return self.state().positions()
