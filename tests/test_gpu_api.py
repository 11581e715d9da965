"""Reference API rows outside the fused decode kernel, through the C ABI:

* spectral_score_forward / spectral_value_forward (sc_block_scores,
  sc_block_values) against the oracle's restatements of
  kernels/spectral_attention.py:375-453 and :544-601;
* get_kv (sc_tier_dequant) against the oracle's TierState.get_kv
  (spectral_cache.py:557-612), elementwise;
* sc_tier_append's flags and its device-side ring-overflow status;
* one-token appends and decode calls that never synchronise the host.

Bars: fp16 results within one fp16 ulp of the oracle (at the larger
magnitude) plus 1e-5 absolute: both sides sum the same fp32 products in a
different order, so a result near a rounding boundary may round to the
neighbouring fp16 value, and a result near zero that is the difference of
O(1) terms differs by the fp32 rounding of those terms (~1e-6)."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import cache_from_states, tables
from helpers import random_state, rope_tables
import oracle.attention as oa

pytestmark = pytest.mark.gpu

ABS = 1e-5


def _ulp16(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _within_ulp(got, ref):
    """One fp16 ulp at the larger of the two magnitudes (a result that
    rounds across a power of two lands one ulp of the higher binade away)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.all(np.abs(got - ref) <= _ulp16(np.maximum(np.abs(got), np.abs(ref))) + ABS)


def _worst(got, ref):
    """The element farthest outside the bar, for the failure message."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    excess = np.abs(got - ref) - _ulp16(np.maximum(np.abs(got), np.abs(ref))) - ABS
    i = np.unravel_index(np.argmax(excess), excess.shape)
    return f"at {tuple(int(x) for x in i)}: got {got[i]!r}, oracle {ref[i]!r}"


@pytest.mark.parametrize("geom", [(2, 4, 128, 512, 16, 0), (8, 4, 128, 512, 32, 4096), (4, 2, 64, 100, 24, 37)])
def test_score_forward_matches_oracle(geom):
    from unsloth_spectral import spectral_score_forward
    Hkv, rep, D, T, k, start = geom
    rng = np.random.default_rng(sum(geom))
    B = 2
    coeffs = (rng.standard_normal((Hkv, T, k)) * 1.2).astype(np.float16)
    basis = (rng.standard_normal((Hkv, k, D)) / np.sqrt(D)).astype(np.float16)
    Q = rng.standard_normal((B, Hkv * rep, D)).astype(np.float16)
    cos, sin = rope_tables(start + T + 8, D)
    ct, st = tables(cos, sin)
    got = spectral_score_forward(torch.from_numpy(Q).cuda()[:, :, None], torch.from_numpy(coeffs).cuda(),
                                 torch.from_numpy(basis).cuda(), ct, st, start, start + T)
    assert got.shape == (B, Hkv * rep, 1, T) and got.dtype == torch.float16
    got = got[:, :, 0].float().cpu().numpy()
    for b in range(B):
        ref = oa.spectral_score_forward(Q[b], coeffs, basis, cos, sin, start)
        assert _within_ulp(got[b], ref), _worst(got[b], ref)


def test_score_forward_refuses_positions_outside_the_tables():
    from unsloth_spectral import spectral_score_forward
    from unsloth_spectral._lib import SpectralHIPError
    ct, st = tables(*rope_tables(100, 128))
    z = torch.zeros(2, 64, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(SpectralHIPError):
        spectral_score_forward(torch.zeros(1, 8, 1, 128, dtype=torch.float16, device="cuda"), z,
                               torch.zeros(2, 16, 128, dtype=torch.float16, device="cuda"), ct, st, 50, 60)


@pytest.mark.parametrize("geom", [(2, 4, 128, 512, 32), (8, 4, 128, 512, 16), (2, 8, 64, 77, 21)])
def test_value_forward_matches_oracle(geom):
    from unsloth_spectral import spectral_value_forward
    Hkv, rep, D, T, k = geom
    rng = np.random.default_rng(100 + sum(geom))
    B = 3
    coeffs = (rng.standard_normal((Hkv, T, k)) * 1.2).astype(np.float16)
    basis = (rng.standard_normal((Hkv, k, D)) / np.sqrt(D)).astype(np.float16)
    P = rng.random((B, Hkv * rep, T)).astype(np.float32) ** 4
    P /= P.sum(-1, keepdims=True)
    P16 = P.astype(np.float16)                      # the reference passes probabilities in the model dtype
    got = spectral_value_forward(torch.from_numpy(P16).cuda()[:, :, None], torch.from_numpy(coeffs).cuda(),
                                 torch.from_numpy(basis).cuda(), D)
    assert got.shape == (B, Hkv * rep, 1, D) and got.dtype == torch.float16
    got = got[:, :, 0].float().cpu().numpy()
    for b in range(B):
        ref = oa.spectral_value_forward(P16[b].astype(np.float32), coeffs, basis)
        assert _within_ulp(got[b], ref), _worst(got[b], ref)


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("ranks", [(16, 32), (32, 32), (64, 16)])
def test_get_kv_matches_oracle(per_row, ranks):
    """cache.get_kv() (sc_tier_dequant for the cold blocks, then the ring in
    order) equals TierState.get_kv: fp16(fp16(code * scale) . basis) with
    fp32 sums, within one fp16 ulp; the tail is copied exactly."""
    kK, kV = ranks
    rng = np.random.default_rng(200 + 10 * per_row + kK + kV)
    states = [random_state(rng, 4, 128, 3, 256, kK, kV, 90, per_row=per_row, batched_qr=True) for _ in range(2)]
    cache = cache_from_states(states, 256)
    K, V = cache.get_kv()
    K, V = K.float().cpu().numpy(), V.float().cpu().numpy()
    for b, s in enumerate(states):
        Kr, Vr = s.get_kv()
        assert K[b].shape == Kr.shape
        assert _within_ulp(K[b], Kr), _worst(K[b], Kr)
        assert _within_ulp(V[b], Vr), _worst(V[b], Vr)
        np.testing.assert_array_equal(K[b, :, 768:], s.tail_k.astype(np.float32))


def _append_raw(cache, K, V, pos, flags):
    """sc_tier_append through the C ABI on the cache's own tiers."""
    from unsloth_spectral import _lib
    lib = _lib.load()
    return lib.sc_tier_append(ctypes.byref(cache._tier()), _lib.ptr(K), _lib.ptr(V), K.stride(0), K.stride(1),
                              K.stride(2), _lib.ptr(pos), K.shape[2], flags, _lib.stream_of(K))


def test_append_overflow_sets_status_and_writes_nothing():
    from unsloth_spectral import SpectralCache, _lib
    cache = SpectralCache(2, 64, block_size=64, k_rank_keys=8, k_rank_values=8, device="cuda", batch_size=2,
                          tail_capacity=128)
    g = torch.Generator(device="cuda").manual_seed(3)
    K = torch.randn(2, 2, 100, 64, generator=g, device="cuda").half()
    assert _append_raw(cache, K, K, None, 0) == 0           # 100 of 128 slots: fits, no compression call
    torch.cuda.synchronize()
    before_k, before_pos = cache.tail_k.clone(), cache.tail_pos.clone()
    K2 = torch.randn(2, 2, 40, 64, generator=g, device="cuda").half()
    assert _append_raw(cache, K2, K2, None, 0) == 0         # 140 > 128: refused on the device, no fault
    torch.cuda.synchronize()
    cnt = cache.counters.cpu().numpy()
    assert (cnt[:, _lib.SC_CNT_STATUS] == _lib.SC_ERR_CAPACITY).all()
    assert (cnt[:, _lib.SC_CNT_TAIL_LEN] == 100).all() and (cnt[:, _lib.SC_CNT_TOTAL] == 100).all()
    assert torch.equal(cache.tail_k, before_k) and torch.equal(cache.tail_pos, before_pos)
    # a reset clears the status and the next append fits again
    assert _append_raw(cache, K2, K2, None, _lib.SC_APPEND_RESET) == 0
    torch.cuda.synchronize()
    cnt = cache.counters.cpu().numpy()
    assert (cnt[:, _lib.SC_CNT_STATUS] == 0).all() and (cnt[:, _lib.SC_CNT_TAIL_LEN] == 40).all()
    assert torch.equal(cache.tail_k[:, :, :40], K2)
    # short appends (a decode step's tokens) take the one-launch path: the
    # same refusal, status and untouched rows
    K4 = torch.randn(2, 2, 87, 64, generator=g, device="cuda").half()
    assert _append_raw(cache, K4, K4, None, 0) == 0          # 127 of 128
    K5 = torch.randn(2, 2, 2, 64, generator=g, device="cuda").half()
    torch.cuda.synchronize()
    before_k = cache.tail_k.clone()
    assert _append_raw(cache, K5, K5, None, 0) == 0          # 129 > 128: refused on the device
    torch.cuda.synchronize()
    cnt = cache.counters.cpu().numpy()
    assert (cnt[:, _lib.SC_CNT_STATUS] == _lib.SC_ERR_CAPACITY).all() and (cnt[:, _lib.SC_CNT_TAIL_LEN] == 127).all()
    assert torch.equal(cache.tail_k, before_k)
    assert _append_raw(cache, K5[:, :, :1], K5[:, :, :1], None, 0) == 0   # 128: fits
    torch.cuda.synchronize()
    assert (cache.counters[:, _lib.SC_CNT_TAIL_LEN] == 128).all()
    assert torch.equal(cache.tail_k[:, :, 127], K5[:, :, 0])
    # a single call larger than the ring is refused on the host
    K3 = torch.zeros(2, 2, 129, 64, dtype=torch.float16, device="cuda")
    assert _append_raw(cache, K3, K3, None, 0) == _lib.SC_ERR_CAPACITY


def test_append_detect_reset_is_per_sequence():
    from unsloth_spectral import SpectralCache, _lib
    cache = SpectralCache(2, 64, block_size=64, k_rank_keys=8, k_rank_values=8, device="cuda", batch_size=2,
                          tail_capacity=256)
    K = torch.ones(2, 2, 30, 64, dtype=torch.float16, device="cuda")
    pos = torch.arange(30, dtype=torch.int32, device="cuda")[None].repeat(2, 1).contiguous()
    assert _append_raw(cache, K, K, pos, _lib.SC_APPEND_DETECT_RESET) == 0
    K1 = torch.full((2, 2, 5, 64), 2.0, dtype=torch.float16, device="cuda")
    pos1 = torch.tensor([[30, 31, 32, 33, 34], [0, 1, 2, 3, 4]], dtype=torch.int32, device="cuda")
    assert _append_raw(cache, K1, K1, pos1, _lib.SC_APPEND_DETECT_RESET) == 0   # sequence 1 restarts
    torch.cuda.synchronize()
    cnt = cache.counters.cpu().numpy()
    assert cnt[0, _lib.SC_CNT_TAIL_LEN] == 35 and cnt[0, _lib.SC_CNT_NEXT_POS] == 35
    assert cnt[1, _lib.SC_CNT_TAIL_LEN] == 5 and cnt[1, _lib.SC_CNT_NEXT_POS] == 5
    assert cache.tail_pos[1, :5].tolist() == [0, 1, 2, 3, 4]
    assert torch.equal(cache.tail_k[1, :, :5], K1[1])
    # without the flag the same positions are appended as given, no reset
    assert _append_raw(cache, K1, K1, pos1, 0) == 0
    torch.cuda.synchronize()
    assert cache.counters[1, _lib.SC_CNT_TAIL_LEN].item() == 10


def test_host_detects_new_generation_from_host_positions():
    """Positions given on the host (or in a multi-token device tensor) are
    compared on the host (spectral_cache.py:177-189); host and device
    counters stay equal."""
    from unsloth_spectral import SpectralCache, _lib
    cache = SpectralCache(2, 128, block_size=128, device="cuda")
    K = torch.randn(1, 2, 200, 128, device="cuda").half()
    cache.append(K, K, list(range(200)))
    cache.append(K[:, :, :1], K[:, :, :1], [200])
    assert cache.total_tokens == 201
    cache.append(K[:, :, :1], K[:, :, :1], [0])                 # host position went backwards: new generation
    assert cache.total_tokens == 1 and cache.num_cold_blocks == 0 and cache.hot_len == 1
    cnt = cache.counters.cpu().numpy()[0]
    assert cnt[_lib.SC_CNT_TOTAL] == 1 and cnt[_lib.SC_CNT_TAIL_LEN] == 1 and cnt[_lib.SC_CNT_NCOLD] == 0
    cache.append(K, K, torch.arange(0, 200, device="cuda")[None])   # multi-token device positions: read
    assert cache.total_tokens == 200 and cache.counters[0, _lib.SC_CNT_TOTAL].item() == 200


def test_one_token_decode_steps_do_not_synchronise():
    """Append of one token with device positions, compression at the block
    boundary and the decode call, under torch's sync debug mode "error":
    no device-to-host synchronisation anywhere on the step."""
    from unsloth_spectral import SpectralCache, _lib
    from unsloth_spectral._decode import run_decode
    H, D, T = 8, 128, 128
    cache = SpectralCache(H, D, block_size=T, k_rank_keys=16, k_rank_values=16, device="cuda", batch_size=2)
    cache.reserve(4 * T)
    g = torch.Generator(device="cuda").manual_seed(9)
    X = torch.randn(2, H, 2 * T + 20, D, generator=g, device="cuda").half()
    cache.append(X[:, :, :T + 100], X[:, :, :T + 100], torch.arange(T + 100, device="cuda")[None].expand(2, -1))
    cos, sin = tables(*rope_tables(4 * T, D))
    Q = torch.randn(2, 4 * H, 1, D, generator=g, device="cuda").half()
    steps = torch.arange(T + 100, 2 * T + 20, device="cuda")
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for i in range(T + 100, 2 * T + 20):   # crosses the block boundary at 2 T
            p = steps[i - T - 100:i - T - 99]
            cache.append(X[:, :, i:i + 1], X[:, :, i:i + 1], p[None].expand(2, 1))
            out = run_decode(Q, cache, cos, sin, p, rope_mode=_lib.SC_ROPE_ABSOLUTE, halves_equal=True)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert cache.num_cold_blocks == 2 and cache.hot_len == 20
    cnt = cache.counters.cpu().numpy()
    assert (cnt[:, _lib.SC_CNT_NCOLD] == 2).all() and (cnt[:, _lib.SC_CNT_TAIL_LEN] == 20).all()
    assert torch.isfinite(out.float()).all()
