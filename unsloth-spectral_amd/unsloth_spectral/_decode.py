"""Host side of the fused decode-attention kernel (sc_decode_attn).

Shared by ``spectral_attention_forward`` (distance RoPE) and
``spectral_attention_decode`` (absolute RoPE).  One call = one launch of the
split-K partial kernel plus one combine launch on the current stream; no
host synchronisation except a one-time check per RoPE table that its two
halves are equal (HF tables are ``cat(freqs, freqs)``), which lets the
kernel read half rows.
"""
import ctypes
import math

import torch

from . import _lib
from ._lib import check, ptr
from .spectral_cache import SpectralCache

_halves = {}


def _halves_equal(cos, sin):
    """Whether both tables have equal halves (HF tables are cat(freqs,
    freqs)); checked once per table pair and version.  The cache entry holds
    weak references to the tables: an entry is used only while both of its
    tables are alive and are the very tensors asked about, so a new table
    that reuses a freed table's memory is checked afresh."""
    import weakref
    key = (cos.data_ptr(), sin.data_ptr(), tuple(cos.shape), cos._version, sin._version)
    hit = _halves.get(key)
    if hit is not None and hit[0]() is cos and hit[1]() is sin:
        return hit[2]
    h = cos.shape[-1] // 2
    eq = bool(torch.equal(cos[:, :h], cos[:, h:]) and torch.equal(sin[:, :h], sin[:, h:]))
    if len(_halves) > 64:
        _halves.clear()
    _halves[key] = (weakref.ref(cos), weakref.ref(sin), eq)
    return eq


def _as_table(t, D):
    if t.dtype != torch.float16:
        t = t.to(torch.float16)
    if t.dim() != 2 or t.shape[-1] != D:
        raise ValueError(f"RoPE table must be [max_len, {D}], got {tuple(t.shape)}")
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def as_cache(cache):
    """Our SpectralCache, or a reference-style object converted once."""
    if isinstance(cache, SpectralCache):
        return cache
    blocks, hk, hv = cache.get_spectral_components()
    return SpectralCache.from_components(blocks, hk, hv, getattr(cache, "hot_position_ids", None),
                                         num_heads=cache.num_heads)


def run_decode(Q, cache, cos, sin, query_position, attention_mask=None, scale=None,
               rope_mode=_lib.SC_ROPE_ABSOLUTE, logits=None, halves_equal=None, split=0):
    """Q [B, Hq, 1, D] post-RoPE query -> [B, Hq, 1, D] in Q.dtype.

    ``logits`` (optional fp32 [B, Hq, T_total]) receives score*scale in cache
    order.  ``attention_mask`` is a keep-mask broadcastable to [B, Hq, 1, T]
    (entries equal to 0 are dropped, spectral_attention.py:284-285).
    ``split`` = workgroups per cold block (0 = chosen from the grid size)."""
    _lib.require_device(Q, "Q")
    if Q.dim() != 4 or Q.shape[2] != 1:
        raise ValueError(f"decode attention takes one query token: Q must be [B, H, 1, D], got {tuple(Q.shape)}")
    cache = as_cache(cache)
    B, Hq, _, D = Q.shape
    if cache._B is None or cache._B != B:
        raise ValueError(f"cache holds {cache._B} sequences, Q has batch {B}")
    if D != cache.head_dim:
        raise ValueError(f"head_dim mismatch: Q {D} vs cache {cache.head_dim}")
    if Hq % cache.num_heads:
        raise ValueError(f"query heads {Hq} not a multiple of KV heads {cache.num_heads}")
    total = cache._n_cold * cache.block_size + cache._tail_len
    if total == 0:
        raise ValueError("Empty cache - no keys available")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if Q.dtype != torch.float16:
        raise NotImplementedError("the HIP decode kernel takes float16 queries (got %s)" % Q.dtype)
    q = Q.reshape(B, Hq, D)
    if q.stride(-1) != 1 or q.stride(1) % 8 or q.stride(0) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    out = torch.empty(B, Hq, 1, D, dtype=torch.float16, device=Q.device)

    a = _lib.ScDecodeArgs()
    tier = cache._tier()
    a.tier = cache._tier_ptr()
    a.q_heads = Hq
    a.rope_mode = rope_mode
    a.grid_blocks = cache._n_cold
    # a pinned grid (captured decode segments) covers the tail tokens of every
    # replayed step; workgroups past the device's tail length write neutral
    # records
    a.grid_tail = cache._tail_len if cache._grid_tail is None else max(cache._tail_len, cache._grid_tail)
    a.scale = float(scale)
    a.split = int(split)
    a.q = q.data_ptr()
    a.q_stride_b, a.q_stride_h = q.stride(0), q.stride(1)
    keep = []
    if rope_mode != _lib.SC_ROPE_NONE:
        cos16 = _as_table(cos, D)
        sin16 = _as_table(sin, D)
        if cos16.stride(0) != sin16.stride(0):
            cos16, sin16 = cos16.contiguous(), sin16.contiguous()
        a.cos, a.sin = cos16.data_ptr(), sin16.data_ptr()
        a.rope_stride = cos16.stride(0)
        a.rope_len = min(cos16.shape[0], sin16.shape[0])
        a.halves_equal = int(_halves_equal(cos16, sin16) if halves_equal is None else halves_equal)
        keep += [cos16, sin16]
    if isinstance(query_position, torch.Tensor):
        qp = query_position.reshape(-1)
        if qp.dtype == torch.int64 and qp.device == Q.device and qp.numel() == B and (B == 1 or qp.stride(0) == 1):
            a.query_pos_i64 = 1          # a model's position ids as they are (no conversion launch)
        else:
            qp = qp.to(device=Q.device, dtype=torch.int32)
            qp = qp.expand(B).contiguous() if qp.numel() == 1 else qp.contiguous()
        a.query_pos = qp.data_ptr()
        keep.append(qp)
    else:
        a.query_pos_scalar = int(query_position)
    if attention_mask is not None:
        m = attention_mask
        if m.dim() == 4:
            m = m[:, :, -1, :]
        m = (m != 0).to(torch.uint8)
        if m.dim() == 2:
            m = m[:, None, :]
        m = m.expand(B, Hq, m.shape[-1])
        if m.shape[-1] < total:
            raise ValueError(f"attention_mask covers {m.shape[-1]} keys, cache holds {total}")
        L = (total + 3) // 4 * 4
        mm = torch.zeros(B, Hq, L, dtype=torch.uint8, device=Q.device)
        mm[:, :, :total] = m[:, :, :total]
        a.mask = mm.data_ptr()
        a.mask_stride_b, a.mask_stride_h = mm.stride(0), mm.stride(1)
        keep.append(mm)
    a.out = out.data_ptr()
    a.out_stride_b, a.out_stride_h = out.stride(0), out.stride(1)
    if logits is not None:
        if logits.dtype != torch.float32 or logits.shape[-1] < total or logits.stride(-1) != 1:
            raise ValueError("logits must be float32 [B, Hq, >= T_total] with unit inner stride")
        a.logits_out = logits.data_ptr()
        a.logits_stride_b, a.logits_stride_h = logits.stride(0), logits.stride(1)
    lib = _lib.load()
    nbytes = ctypes.c_size_t(0)
    check(lib.sc_decode_workspace_size(ctypes.byref(a), ctypes.byref(nbytes)))
    ws = _lib.workspace(Q.device, nbytes.value)
    check(lib.sc_decode_attn(ctypes.byref(a), ptr(ws), ws.numel(), _lib.stream_of(Q)))
    return out if Q.dtype == torch.float16 else out.to(Q.dtype)
