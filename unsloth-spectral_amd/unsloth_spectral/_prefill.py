"""Prefill attention over the spectral tiers (HIP kernel sc_prefill_attn).

A chunk of T query tokens per sequence attends over the cache's cold blocks
and FP16 tail with a causal mask (key position <= query position), keys
rotated at their absolute positions with apply_rope's first-half cos/sin
(integration.py:292-346 reconstructs everything with get_kv and runs dense
attention; the kernel reconstructs 16-token tiles on the fly instead)."""
import ctypes
import math

import torch

from . import _lib
from ._lib import check


def prefill_supported(cache, q_heads):
    return cache.head_dim == 128 and q_heads == 4 * cache.num_heads and cache.block_size % 16 == 0


def run_prefill(q, cache, cos, sin, position_ids, scale=None):
    """q [B, Hq, T, 128] fp16 post-RoPE query; position_ids [B, T] (or [1, T])
    absolute positions; cos/sin [L, 128] RoPE tables covering every cached
    position.  Returns [B, Hq, T, 128] fp16."""
    _lib.require_device(q, "q")
    if q.dim() != 4 or q.dtype != torch.float16:
        raise ValueError(f"q must be float16 [B, H, T, D], got {q.dtype} {tuple(q.shape)}")
    B, Hq, T, D = q.shape
    if cache._B is None or cache._B != B:
        raise ValueError(f"cache holds {cache._B} sequences, q has batch {B}")
    if not prefill_supported(cache, Hq):
        raise NotImplementedError("prefill kernel: head_dim 128 and 4 query heads per KV head")
    if q.stride(-1) != 1 or q.stride(2) % 8 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    pos = position_ids.to(device=q.device, dtype=torch.int32).reshape(-1, T)
    pos = pos.expand(B, T).contiguous() if pos.shape[0] != B else pos.contiguous()
    cos16 = cos.to(device=q.device, dtype=torch.float16)
    sin16 = sin.to(device=q.device, dtype=torch.float16)
    if cos16.stride(-1) != 1 or cos16.stride(0) % 4 or cos16.data_ptr() % 8:
        cos16 = cos16.contiguous()
    if sin16.stride() != cos16.stride() or sin16.data_ptr() % 8:
        sin16, cos16 = sin16.contiguous(), cos16.contiguous()
    out = torch.empty(B, Hq, T, D, dtype=torch.float16, device=q.device)
    a = _lib.ScPrefillArgs()
    tier = cache._tier()
    a.tier = ctypes.pointer(tier)
    a.q_heads, a.t_q = Hq, T
    a.scale = float(scale if scale is not None else 1.0 / math.sqrt(D))
    a.q, a.q_stride_b, a.q_stride_h, a.q_stride_t = q.data_ptr(), q.stride(0), q.stride(1), q.stride(2)
    a.query_pos, a.query_pos_stride_b = pos.data_ptr(), pos.stride(0)
    a.cos, a.sin, a.rope_stride = cos16.data_ptr(), sin16.data_ptr(), cos16.stride(0)
    a.rope_len = min(cos16.shape[0], sin16.shape[0])
    a.out, a.out_stride_b, a.out_stride_h, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1), \
        out.stride(2)
    check(_lib.load().sc_prefill_attn(ctypes.byref(a), _lib.stream_of(q)))
    return out
