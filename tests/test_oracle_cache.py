"""Pins the tier-manager restatement (oracle/cache.py) with the reference's
own tier-count assertions and invariants.

COLAB_LONG_CONTEXT_VALIDATION.py:255-275 asserts 100 tokens -> 0 blocks and
600 tokens -> 1 block + 88 hot; test_gqa_fix.py:93-94 asserts KV-head counts
of the blocks; spectral_cache.py:176-189 resets on a backwards position."""
import numpy as np

from oracle.cache import TierManager


def _omega(seed=0):
    rng = np.random.default_rng(seed)
    return lambda kind, idx, shape: rng.standard_normal(shape).astype(np.float32)


def _kv(rng, H, T, D):
    return rng.standard_normal((H, T, D)).astype(np.float16), rng.standard_normal((H, T, D)).astype(np.float16)


def test_tier_counts_match_reference_assertions():
    rng = np.random.default_rng(0)
    tm = TierManager(8, 128, omega_fn=_omega())
    tm.append(*_kv(rng, 8, 100, 128), np.arange(100))
    assert len(tm.blocks) == 0 and tm.hot_K.shape[1] == 100
    tm2 = TierManager(8, 128, omega_fn=_omega())
    tm2.append(*_kv(rng, 8, 600, 128), np.arange(600))
    assert len(tm2.blocks) == 1 and tm2.hot_K.shape[1] == 88
    assert tm2.blocks[0].codes_k.shape == (8, 512, 16) and tm2.blocks[0].codes_v.shape == (8, 512, 32)
    np.testing.assert_array_equal(tm2.get_all_positions(), np.arange(600))


def test_while_loop_compresses_every_full_block():
    rng = np.random.default_rng(1)
    tm = TierManager(2, 64, block_size=128, k_rank_keys=8, k_rank_values=8, omega_fn=_omega())
    for s in range(0, 1000, 250):
        tm.append(*_kv(rng, 2, 250, 64), np.arange(s, s + 250))
    assert len(tm.blocks) == 7 and tm.hot_K.shape[1] == 1000 - 7 * 128
    assert [b.start for b in tm.blocks] == [128 * j for j in range(7)]
    assert tm.compression_count == 7 and tm.total_tokens == 1000


def test_exact_block_leaves_empty_tail():
    rng = np.random.default_rng(2)
    tm = TierManager(2, 64, block_size=128, k_rank_keys=8, k_rank_values=8, omega_fn=_omega())
    tm.append(*_kv(rng, 2, 128, 64), np.arange(128))
    assert len(tm.blocks) == 1 and tm.hot_K is None


def test_new_generation_resets():
    rng = np.random.default_rng(3)
    tm = TierManager(2, 64, block_size=128, k_rank_keys=8, k_rank_values=8, omega_fn=_omega())
    tm.append(*_kv(rng, 2, 300, 64), np.arange(300))
    assert len(tm.blocks) == 2
    tm.append(*_kv(rng, 2, 5, 64), np.arange(5))        # positions restart
    assert len(tm.blocks) == 0 and tm.total_tokens == 5 and tm.hot_K.shape[1] == 5


def test_get_kv_reconstructs_low_rank_blocks():
    rng = np.random.default_rng(4)
    H, T, D, r = 2, 128, 64, 6
    A = (rng.standard_normal((H, T, r)) @ rng.standard_normal((H, r, D))).astype(np.float16)
    tm = TierManager(H, D, block_size=T, k_rank_keys=8, k_rank_values=8, omega_fn=_omega())
    tm.append(A, A, np.arange(T))
    K, V = tm.state().get_kv()
    rel = np.linalg.norm(K.astype(np.float64) - A) / np.linalg.norm(A.astype(np.float64))
    assert rel < 1e-2          # INT8 coefficient quantisation only
