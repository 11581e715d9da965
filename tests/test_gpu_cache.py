"""Tier manager on the GPU vs the oracle tier manager (counts, positions,
tail contents, reset) and decode over tiers built by appends."""
import numpy as np
import pytest
import torch

from gpu_helpers import export_states, tables
from helpers import pearson, rope_tables
from oracle.attention import spectral_attention_decode as o_abs
from oracle.attention import spectral_attention_forward as o_dist
from oracle.cache import TierManager

pytestmark = pytest.mark.gpu


def _omega(seed=0):
    rng = np.random.default_rng(seed)
    return lambda kind, idx, shape: rng.standard_normal(shape).astype(np.float32)


def _make(H=2, D=128, T=128, kK=16, kV=32, B=1, **kw):
    from unsloth_spectral import SpectralCache
    return SpectralCache(H, D, block_size=T, k_rank_keys=kK, k_rank_values=kV, device="cuda", **kw)


def test_append_counts_positions_and_tail_match_oracle():
    rng = np.random.default_rng(0)
    H, D, T = 2, 128, 128
    cache = _make(H, D, T, max_blocks=2, tail_capacity=256)
    tm = TierManager(H, D, block_size=T, k_rank_keys=16, k_rank_values=32, omega_fn=_omega())
    pos = 0
    for n in (50, 50, 1, 27, 300, 1, 1, 128, 64, 200, 3):
        K = rng.standard_normal((1, H, n, D)).astype(np.float16)
        V = rng.standard_normal((1, H, n, D)).astype(np.float16)
        p = np.arange(pos, pos + n)
        cache.append(torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda(), torch.from_numpy(p).cuda()[None])
        tm.append(K[0], V[0], p)
        pos += n
        assert cache.total_tokens == tm.total_tokens
        assert cache.num_cold_blocks == len(tm.blocks)
        assert cache.compression_count == tm.compression_count
        if tm.hot_K is None:
            assert cache.hot_K is None
        else:
            np.testing.assert_array_equal(cache.hot_K[0].cpu().numpy(), tm.hot_K)
            np.testing.assert_array_equal(cache.hot_V[0].cpu().numpy(), tm.hot_V)
            np.testing.assert_array_equal(cache.hot_position_ids[0].cpu().numpy(), tm.hot_pos)
        np.testing.assert_array_equal(cache.get_all_positions().cpu().numpy(), tm.get_all_positions())
    cnt = cache.counters.cpu().numpy()[0]
    assert cnt[0] == cache.num_cold_blocks and cnt[2] == cache.hot_len and cnt[4] == cache.total_tokens
    assert [b.start_position for b in cache.cold_blocks] == [b.start for b in tm.blocks]


def test_int64_and_int32_positions_append_the_same_tiers():
    """int64 position ids go to the append kernel as they are
    (SC_APPEND_POS_I64); int32 ones, and int64 views that are not
    contiguous, through the int32 array: the same tail rows, positions and
    counters, including a device-detected new generation."""
    rng = np.random.default_rng(5)
    H, D, T = 2, 128, 128
    caches = [_make(H, D, T, tail_capacity=512) for _ in range(3)]
    for n, start in ((40, 0), (1, 40), (1, 41), (30, 7), (1, 37)):
        K = torch.from_numpy(rng.standard_normal((2, H, n, D)).astype(np.float16)).cuda()
        V = torch.from_numpy(rng.standard_normal((2, H, n, D)).astype(np.float16)).cuda()
        p64 = torch.arange(start, start + n, device="cuda")[None].expand(2, n).contiguous()
        wide = torch.stack([p64, p64], dim=-1)[..., 0]                       # int64, not contiguous
        for c, p in zip(caches, (p64, p64.to(torch.int32), wide)):
            c.append(K, V, p)
    for c in caches[1:]:
        assert torch.equal(c.counters, caches[0].counters)
        assert torch.equal(c.tail_k, caches[0].tail_k) and torch.equal(c.tail_pos, caches[0].tail_pos)
        assert c.total_tokens == caches[0].total_tokens and c.hot_len == caches[0].hot_len
    assert caches[0].hot_position_ids[0].tolist() == list(range(7, 38))


def test_low_rank_blocks_reconstruct():
    rng = np.random.default_rng(1)
    H, D, T, r = 2, 128, 128, 6
    A = (rng.standard_normal((1, H, 3 * T, r)) @ rng.standard_normal((1, H, r, D))).astype(np.float16)
    cache = _make(H, D, T, quant_granularity="per_row")
    At = torch.from_numpy(A).cuda()
    cache.append(At, At)
    K, V = cache.get_kv()
    assert K.shape == (1, H, 3 * T, D)
    rel = (K.float() - At.float()).norm() / At.float().norm()
    assert rel.item() < 5e-3


def test_new_generation_resets_on_device_and_host():
    rng = np.random.default_rng(2)
    cache = _make(2, 128, 128)
    for start in (0, 0):
        K = torch.from_numpy(rng.standard_normal((1, 2, 300, 128)).astype(np.float16)).cuda()
        cache.append(K, K, torch.arange(start, start + 300, device="cuda")[None])
    assert cache.total_tokens == 300 and cache.num_cold_blocks == 2 and cache.hot_len == 44
    cnt = cache.counters.cpu().numpy()[0]
    assert cnt[4] == 300 and cnt[0] == 2 and cnt[2] == 44


def test_ring_wraps_and_grows():
    rng = np.random.default_rng(3)
    cache = _make(2, 64, 64, kK=8, kV=8, tail_capacity=128)
    tm = TierManager(2, 64, block_size=64, k_rank_keys=8, k_rank_values=8, omega_fn=_omega())
    pos = 0
    for n in (40, 40, 40, 500, 1, 63, 1, 90):
        K = rng.standard_normal((1, 2, n, 64)).astype(np.float16)
        cache.append(torch.from_numpy(K).cuda(), torch.from_numpy(K).cuda())
        tm.append(K[0], K[0], None)
        pos += n
        if tm.hot_K is not None:
            np.testing.assert_array_equal(cache.hot_K[0].cpu().numpy(), tm.hot_K)
        assert cache.num_cold_blocks == len(tm.blocks)


@pytest.mark.parametrize("unit_scale", [True, False])
@pytest.mark.parametrize("mode", ["absolute", "distance"])
def test_decode_over_appended_tiers(mode, unit_scale):
    """The whole pipeline on the benchmark's data distribution (low rank +
    noise; literal, i.e. noise-dominated, and lifted to unit scale): appends,
    blocks compressed on the device, then attention checked against the
    oracle evaluated on exactly those tiers (exported INT8 codes / scales /
    bases): outputs to the decode bar, logits Pearson >= 0.9999."""
    from unsloth_spectral import _lib
    from unsloth_spectral._decode import run_decode
    rng = np.random.default_rng(4 + unit_scale)
    H, D, T, B = 8, 128, 512, 2
    cache = _make(H, D, T, B=B, kK=16, kV=32)
    from helpers import lowrank_plus_noise
    total = 2 * T + 300
    K = lowrank_plus_noise(rng, B * H, total, D, unit_scale=unit_scale).reshape(B, H, total, D)
    V = lowrank_plus_noise(rng, B * H, total, D, unit_scale=unit_scale).reshape(B, H, total, D)
    for s in range(0, total, 200):
        e = min(total, s + 200)
        cache.append(torch.from_numpy(K[:, :, s:e]).cuda(), torch.from_numpy(V[:, :, s:e]).cuda(),
                     torch.arange(s, e, device="cuda")[None].expand(B, -1))
    assert cache.num_cold_blocks == 2 and cache.hot_len == 300
    states = export_states(cache)
    cos, sin = rope_tables(total + 8, D)
    ct, st = tables(cos, sin)
    Q = rng.standard_normal((B, 4 * H, 1, D)).astype(np.float16)
    code, ofn = (_lib.SC_ROPE_ABSOLUTE, o_abs) if mode == "absolute" else (_lib.SC_ROPE_DISTANCE, o_dist)
    logits = torch.full((B, 4 * H, total), float("nan"), dtype=torch.float32, device="cuda")
    out = run_decode(torch.from_numpy(Q).cuda(), cache, ct, st, total - 1, rope_mode=code, logits=logits)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    for b in range(B):
        ref, _, logits16 = ofn(Q[b, :, 0], states[b], cos, sin, total - 1)
        err = np.abs(out[b, :, 0].float().cpu().numpy() - ref.astype(np.float64)).max()
        assert err < 2e-3 and err < 1e-2 * np.abs(ref.astype(np.float64)).max(), err
        assert np.isfinite(lg[b]).all()
        assert pearson(lg[b].ravel(), logits16.astype(np.float64).ravel()) >= 0.9999
    # the compressed blocks approximate the raw keys like an rSVD of rank 16 should
    # (the literal data are noise-dominated: most of the noise is not in 16 directions)
    Kr, _ = cache.get_kv()
    rel = ((Kr[:, :, :2 * T].float().cpu() - torch.from_numpy(K[:, :, :2 * T]).float()).norm()
           / torch.from_numpy(K[:, :, :2 * T]).float().norm())
    assert rel.item() < (0.2 if unit_scale else 0.9), rel.item()


def test_memory_stats_and_tuple_emulation():
    rng = np.random.default_rng(5)
    cache = _make(2, 128, 128)
    K = torch.from_numpy(rng.standard_normal((1, 2, 300, 128)).astype(np.float16)).cuda()
    cache.append(K, K)
    s = cache.get_memory_stats()
    assert s["num_blocks"] == 2 and s["total_tokens"] == 300 and s["compression_ratio"] > 1
    k0, v0 = cache
    assert k0.shape == (1, 2, 300, 128) and torch.equal(cache[0], k0)
    with pytest.raises(IndexError):
        cache[2]
    assert len(cache) == 300 and "SpectralCache(tokens=300" in repr(cache)
