"""sc_decode_attn_noalloc (records in the library's own device array) against
sc_decode_attn with a caller workspace, through the C ABI.

Two calls in a row, the second with a smaller input, each compared bit for
bit with the workspace entry point on the same inputs; then the size limit:
a call whose records exceed SC_DECODE_SCRATCH_BYTES is refused on the host
with SC_ERR_WORKSPACE before anything is launched."""
import ctypes
import math

import numpy as np
import pytest
import torch

from gpu_helpers import cache_from_states, tables
from helpers import random_state, rope_tables

pytestmark = pytest.mark.gpu


def _args(cache, Q, out, cos, sin, qpos, logits=None):
    from unsloth_spectral import _lib
    a = _lib.ScDecodeArgs()
    tier = cache._tier()
    a.tier = ctypes.pointer(tier)
    B, Hq, D = Q.shape
    a.q_heads, a.rope_mode = Hq, _lib.SC_ROPE_ABSOLUTE
    a.grid_blocks, a.grid_tail = cache.num_cold_blocks, cache.hot_len
    a.scale = 1.0 / math.sqrt(D)
    a.q, a.q_stride_b, a.q_stride_h = Q.data_ptr(), Q.stride(0), Q.stride(1)
    a.cos, a.sin, a.rope_stride, a.rope_len, a.halves_equal = cos.data_ptr(), sin.data_ptr(), D, cos.shape[0], 1
    a.query_pos_scalar = qpos
    a.out, a.out_stride_b, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    if logits is not None:
        a.logits_out = logits.data_ptr()
        a.logits_stride_b, a.logits_stride_h = logits.stride(0), logits.stride(1)
    return a, tier


def _both(states, block_size, seed, with_logits):
    """Outputs (and logits) of sc_decode_attn and of sc_decode_attn_noalloc."""
    from unsloth_spectral import _lib
    lib = _lib.load()
    cache = cache_from_states(states, block_size)
    total = states[0].total_tokens()
    cos, sin = tables(*rope_tables(total + 16, 128))
    B, Hkv = len(states), states[0].num_heads
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.randn(B, 4 * Hkv, 128, generator=g, device="cuda").half()
    res = []
    for noalloc in (False, True):
        out = torch.full((B, 4 * Hkv, 128), float("nan"), dtype=torch.float16, device="cuda")
        lg = torch.full((B, 4 * Hkv, total), float("nan"), device="cuda") if with_logits else None
        a, tier = _args(cache, Q, out, cos, sin, total - 1, lg)
        stream = _lib.stream_of(Q)
        if noalloc:
            _lib.check(lib.sc_decode_attn_noalloc(ctypes.byref(a), stream))
        else:
            n = ctypes.c_size_t(0)
            _lib.check(lib.sc_decode_workspace_size(ctypes.byref(a), ctypes.byref(n)))
            ws = torch.empty(n.value, dtype=torch.uint8, device="cuda")
            _lib.check(lib.sc_decode_attn(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream))
        torch.cuda.synchronize()
        res.append((out.cpu(), None if lg is None else lg.cpu()))
    return res


def test_noalloc_matches_workspace_entry_point_twice_shrinking():
    rng = np.random.default_rng(31)
    big = [random_state(rng, 8, 128, 12, 512, 32, 32, 300, per_row=True) for _ in range(4)]
    small = [random_state(rng, 2, 128, 3, 256, 16, 32, 70) for _ in range(2)]
    for name, states, bs, with_logits in (("big, branch-free path", big, 512, False),
                                          ("small, general path", small, 256, True)):
        print(f"noalloc case: {name}", flush=True)
        (o_ws, l_ws), (o_na, l_na) = _both(states, bs, 5, with_logits)
        assert torch.isfinite(o_ws.float()).all()
        assert torch.equal(o_ws, o_na), name
        if with_logits:
            assert torch.equal(torch.nan_to_num(l_ws, nan=7.0), torch.nan_to_num(l_na, nan=7.0))


def test_noalloc_refuses_records_beyond_its_scratch():
    from unsloth_spectral import SpectralCache, _lib
    lib = _lib.load()
    # batch 1, 8 KV heads, 256 cold slots split 8 ways: 2048 units x 8 heads
    # x 4 query heads x 528 bytes = 34.6 MB of records > 32 MiB
    cache = SpectralCache(8, 128, block_size=512, k_rank_keys=16, k_rank_values=16, device="cuda",
                          batch_size=1, max_blocks=256)
    cos, sin = tables(*rope_tables(64, 128))
    Q = torch.zeros(1, 32, 128, dtype=torch.float16, device="cuda")
    out = torch.empty_like(Q)
    a, tier = _args(cache, Q, out, cos, sin, 0)
    a.grid_blocks, a.split = 256, 8
    n = ctypes.c_size_t(0)
    _lib.check(lib.sc_decode_workspace_size(ctypes.byref(a), ctypes.byref(n)))
    assert n.value > _lib.SC_DECODE_SCRATCH_BYTES, n.value   # checked before the entry point is called
    rc = lib.sc_decode_attn_noalloc(ctypes.byref(a), _lib.stream_of(Q))
    assert rc == -3, rc
    assert b"scratch" in lib.sc_last_error()
