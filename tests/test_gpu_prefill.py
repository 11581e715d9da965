"""Prefill attention over the tiers (sc_prefill_attn) against the float64
closed form: causal softmax attention of each query over every cached key
(cold keys dequantised as fp16(code * scale) . basis, like get_kv, and
every key rotated at its absolute position with apply_rope's first-half
cos/sin, integration.py:292-346), and against the torch restatement of the
reference path (dense fp16 attention over get_kv) on the GPU.

Bar: 2e-3 max-abs and 1e-2 of max|ref| (FP16 out, FP32 accumulate)."""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import cache_from_states, tables
from helpers import random_state, rope_tables

pytestmark = pytest.mark.gpu
ATOL, RTOL_MAX = 2e-3, 1e-2


def _closed_form(Q, state, cos, sin, qpos):
    """Q [Hq, T, D] fp16, qpos [T] -> [Hq, T, D] float64."""
    K, V = state.get_kv()                        # [H, L, D] fp16 (dequantised cold blocks, then the tail)
    pos = np.asarray(state.positions())
    K = K.astype(np.float64)
    V = V.astype(np.float64)
    D = K.shape[-1]
    c = cos[pos, :D // 2].astype(np.float64)[None]
    s = sin[pos, :D // 2].astype(np.float64)[None]
    x1, x2 = K[..., :D // 2], K[..., D // 2:]
    Kr = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    rep = Q.shape[0] // K.shape[0]
    Kr, V = np.repeat(Kr, rep, 0), np.repeat(V, rep, 0)
    lg = np.einsum("htd,hld->htl", Q.astype(np.float64), Kr) / math.sqrt(D)
    lg = np.where(pos[None, None, :] <= np.asarray(qpos)[None, :, None], lg, -np.inf)
    p = np.exp(lg - lg.max(-1, keepdims=True))
    return np.einsum("htl,hld->htd", p / p.sum(-1, keepdims=True), V)


def _check(out, ref):
    err = np.abs(out - ref).max()
    assert err <= ATOL, err
    assert err <= RTOL_MAX * np.abs(ref).max(), (err, np.abs(ref).max())


CASES = [
    # H_kv, nblk, T, kK, kV, tail, per_row, T_q (queries = the last T_q cached tokens)
    (2, 3, 128, 16, 32, 40, False, 40),
    (2, 2, 128, 32, 32, 100, True, 356),       # every cached token queries: a whole-prompt prefill
    (1, 2, 64, 64, 16, 7, True, 17),
    (2, 0, 128, 16, 32, 77, False, 77),        # tail only
    (8, 1, 512, 32, 32, 3, True, 33),
]


@pytest.mark.parametrize("case", CASES)
def test_prefill_matches_closed_form(case):
    from unsloth_spectral._prefill import run_prefill
    H, nblk, T, kK, kV, tail, per_row, Tq = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    B = 2
    states = [random_state(rng, H, 128, nblk, T, kK, kV, tail, per_row=per_row, start=500 * b) for b in range(B)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 1100, 128)
    cache = cache_from_states(states, block_size=T)
    Q = (rng.standard_normal((B, 4 * H, Tq, 128))).astype(np.float16)
    qpos = np.stack([np.asarray(st.positions())[-Tq:] for st in states])
    ct, sn = tables(cos, sin)
    out = run_prefill(torch.from_numpy(Q).cuda(), cache, ct, sn, torch.from_numpy(qpos).cuda())
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    for b in range(B):
        _check(out[b], _closed_form(Q[b], states[b], cos, sin, qpos[b]))


def test_prefill_shuffled_query_positions():
    """Query tokens whose positions are not increasing (each sees the keys at
    or before its own position): masks are decided per query, and the
    fully-visible shortcut only for key tiles before every query of a
    sub-tile."""
    from unsloth_spectral._prefill import run_prefill
    rng = np.random.default_rng(31)
    states = [random_state(rng, 2, 128, 3, 128, 16, 32, 60, per_row=True)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 8, 128)
    cache = cache_from_states(states, block_size=128)
    Tq = 70
    Q = rng.standard_normal((1, 8, Tq, 128)).astype(np.float16)
    qpos = rng.permutation(np.asarray(states[0].positions()))[:Tq][None].astype(np.int32)
    ct, sn = tables(cos, sin)
    out = run_prefill(torch.from_numpy(Q).cuda(), cache, ct, sn, torch.from_numpy(qpos).cuda())
    torch.cuda.synchronize()
    _check(out[0].float().cpu().numpy(), _closed_form(Q[0], states[0], cos, sin, qpos[0]))


@pytest.mark.parametrize("ranks", [(16, 16), (32, 16), (16, 32), (32, 32)])
def test_prefill_rows_do_not_depend_on_the_other_queries(ranks):
    """A query's output is bit-identical whether it is prefilled with the
    whole prompt or in a chunk of its own: the kernel groups consecutive
    queries into workgroups and scans key tiles up to the last query of the
    group, so a query also passes key tiles that are entirely after its own
    position; those must leave its softmax state exactly unchanged.  Queries
    are scaled so that the running maxima reach |m log2(e)| >= 2, where a
    rescale factor computed as exp2 of the rounding error of m log2(e) would
    round to 1 +- 2^-23 instead of 1."""
    from unsloth_spectral._prefill import run_prefill
    rng = np.random.default_rng(41)
    states = [random_state(rng, 8, 128, 2, 512, ranks[0], ranks[1], 200, per_row=True)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 16, 128)
    ct, sn = tables(cos, sin)
    cache = cache_from_states(states, block_size=512)
    Q = torch.from_numpy((4.0 * rng.standard_normal((1, 32, total, 128))).astype(np.float16)).cuda()
    pos = torch.arange(total, device="cuda")[None]
    full = run_prefill(Q, cache, ct, sn, pos)
    for a, b in ((0, 37), (5, 42), (300, 301), (700, 813), (total - 53, total)):
        part = run_prefill(Q[:, :, a:b].contiguous(), cache, ct, sn, pos[:, a:b].contiguous())
        torch.cuda.synchronize()
        diff = int((part != full[:, :, a:b]).sum())
        assert diff == 0, f"queries {a}:{b}: {diff} outputs differ from the whole-prompt prefill"


def test_prefill_matches_dense_reference_path():
    """Against integration._dense_prefill (dense fp16 attention over get_kv,
    the reference's own prefill arithmetic) on the GPU."""
    from unsloth_spectral._prefill import run_prefill
    from unsloth_spectral.integration import _dense_prefill
    rng = np.random.default_rng(21)
    states = [random_state(rng, 8, 128, 2, 512, 32, 32, 200, per_row=True)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 16, 128)
    ct, sn = tables(cos, sin)
    cache = cache_from_states(states, block_size=512)
    Tq = 300
    Q = torch.from_numpy(rng.standard_normal((1, 32, Tq, 128)).astype(np.float16)).cuda()
    qpos = torch.arange(total - Tq, total, device="cuda")[None]
    got = run_prefill(Q, cache, ct, sn, qpos)
    ref = _dense_prefill(Q, cache, ct, sn, 4, None, 1.0 / math.sqrt(128), qpos)
    torch.cuda.synchronize()
    _check(got.float().cpu().numpy(), ref.float().cpu().numpy())


def test_prefill_rejects_unsupported_geometry():
    from unsloth_spectral._lib import SpectralHIPError
    from unsloth_spectral._prefill import run_prefill
    from unsloth_spectral import _lib
    import ctypes
    rng = np.random.default_rng(3)
    states = [random_state(rng, 2, 128, 1, 128, 16, 16, 10)]
    cache = cache_from_states(states, block_size=128)
    cos, sin = tables(*rope_tables(200, 128))
    with pytest.raises(NotImplementedError):   # GQA group 2: the wrapper refuses before the ABI
        run_prefill(torch.zeros(1, 4, 3, 128, dtype=torch.float16, device="cuda"), cache, cos, sin,
                    torch.arange(3, device="cuda")[None])
    a = _lib.ScPrefillArgs()                   # and the ABI itself says why
    tier = cache._tier()
    a.tier = ctypes.pointer(tier)
    a.q_heads, a.t_q = 4, 3
    with pytest.raises(SpectralHIPError, match="GQA"):
        _lib.check(_lib.load().sc_prefill_attn(ctypes.byref(a), None))
