"""Model integration: per-layer spectral cache behind the attention module.

API of unsloth_spectral/integration.py: ``create_spectral_forward``
(:43-425), ``apply_rotary_pos_emb`` (:428-465), ``repeat_kv`` (:468-478),
``create_spectral_forward_inference`` (:481-725), ``patch_unsloth_attention``
(:728-889), ``get_cache_stats`` (:892-938).

Order of operations per layer and step (integration.py:596-659): project
Q/K/V, rotate Q (and K for the dense prefill), append the *pre-RoPE* K and V
to the layer's SpectralCache (compression fires inside append), then attend.
One-token decode steps run the fused HIP kernel over all tiers (cold blocks
and FP16 tail, so the reference's ``total_tokens > block_size`` branch and
its dense fallback are the same kernel with zero or more cold blocks).
Multi-token (prefill) steps attend causally over every tier with the HIP
prefill kernel (tiles reconstructed on the fly); the reference's dense
attention over ``get_kv`` (:292-346) remains for geometries the kernel does
not take and for ``use_spectral_attention=False``.

The patched forward accepts the attention signature of transformers 5.x
(``position_embeddings=(cos, sin)`` for the current tokens, cache in the
module) and keeps each layer's SpectralCache on the module; full RoPE
tables for the cached positions come from the model's rotary module.
"""
import logging
import math
from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib
from ._decode import run_decode
from ._prefill import prefill_supported, run_prefill
from .spectral_attention import apply_rope, repeat_kv as _repeat_kv
from .spectral_cache import SpectralCache

logger = logging.getLogger("unsloth_spectral.integration")

TRITON_KERNELS_AVAILABLE = False


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _rotate_queries(q, cos, sin):
    """``q * cos + rotate_half(q) * sin`` for q [B, H, T, D] and cos/sin
    [B, T, D] or [T, D] (integration.py:610-613 with :428-465), as fp16.
    fp16 operands with 16-byte rows go to sc_rope_rotate: one launch instead
    of five elementwise ops, bit-identical to the fp16 tensor expression.
    Other dtypes or layouts use the tensor expression."""
    B, H, T, D = q.shape
    if cos.dim() == 2:
        cos, sin = cos[None], sin[None]
    ok = (q.dtype == cos.dtype == sin.dtype == torch.float16 and q.is_cuda and D % 16 == 0 and D <= 256
          and cos.shape[1:] == (T, D) and cos.shape[0] in (1, B) and sin.shape == cos.shape
          and cos.stride() == sin.stride() and q.stride(-1) == 1 and cos.stride(-1) == 1
          and all(s % 8 == 0 for s in q.stride()[:3] + cos.stride()[:2])
          and q.data_ptr() % 16 == 0 and cos.data_ptr() % 16 == 0 and sin.data_ptr() % 16 == 0)
    if not ok:
        return (q * cos[:, None] + rotate_half(q) * sin[:, None]).to(torch.float16)
    out = torch.empty(B, H, T, D, dtype=torch.float16, device=q.device)
    cb = cos.stride(0) if cos.shape[0] == B and B > 1 else 0
    _lib.check(_lib.load().sc_rope_rotate(
        _lib.ptr(q), q.stride(0), q.stride(1), q.stride(2), _lib.ptr(cos), _lib.ptr(sin), cb, cos.stride(1),
        B, H, T, D, _lib.ptr(out), _lib.stream_of(q)))
    return out


def apply_rotary_pos_emb(q, k, cos, sin, position_ids=None):
    """HF rotate_half RoPE (integration.py:428-465); cos/sin [T, D] or [B, T, D]."""
    if cos.dim() == 2:
        cos, sin = cos[None, None], sin[None, None]
    elif cos.dim() == 3:
        cos, sin = cos[:, None], sin[:, None]
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    return _repeat_kv(hidden_states, n_rep)


class _RopeTable:
    """Full cos/sin tables [L, D] (fp16) for absolute positions, built with
    the model's own rotary module so the values equal what the model uses."""

    def __init__(self, rotary, head_dim, theta=None):
        self.rotary = rotary
        self.head_dim = head_dim
        self.theta = theta
        self.cos = None
        self.sin = None

    def get(self, length, device):
        if self.cos is None or self.cos.shape[0] < length or self.cos.device != device:
            L = 1 << max(12, (int(length) - 1).bit_length())
            pos = torch.arange(L, device=device)
            if self.rotary is not None:
                dummy = torch.zeros(1, 1, self.head_dim, dtype=torch.float16, device=device)
                c, s = self.rotary(dummy, pos[None])
                c, s = c[0], s[0]
            else:
                inv = 1.0 / (self.theta ** (torch.arange(0, self.head_dim, 2, device=device).float()
                                            / self.head_dim))
                emb = torch.cat([torch.outer(pos.float(), inv)] * 2, dim=-1)
                c, s = emb.cos(), emb.sin()
            self.cos = c.to(torch.float16).contiguous()
            self.sin = s.to(torch.float16).contiguous()
        return self.cos, self.sin


def _model_rope(module, head_dim):
    tab = getattr(module, "_spectral_rope", None)
    if tab is None:
        theta = getattr(getattr(module, "config", None), "rope_theta", None) or 10000.0
        tab = _RopeTable(getattr(module, "rotary_emb", None), head_dim, theta)
        module._spectral_rope = tab
    return tab


def _dense_prefill(q_rot, cache, cos_tab, sin_tab, n_rep, key_keep, scale, q_pos, rows=1024):
    """Dense attention over get_kv() with keys rotated at their absolute
    positions (integration.py:297-346): fp16 scores, softmax in fp32 cast
    back to fp16, fp16 P.V.  Causality comes from each sequence's positions
    (key position <= query position), so a prompt appended in several chunks
    sees the right keys; ``key_keep`` ([B, L] flags, 1 = attend, or None)
    drops padding keys.  Query rows are processed in slices of ``rows`` to
    bound the [Hq, rows, L] score buffer.  Both products take contiguous
    operands."""
    K, V = cache.get_kv()
    pos = cache.positions()                                  # [B, L]
    K = apply_rope(K, cos_tab[pos][:, None], sin_tab[pos][:, None])
    Kt = _repeat_kv(K, n_rep).transpose(2, 3).contiguous()
    V = _repeat_kv(V, n_rep).contiguous()
    B, T = q_rot.shape[0], q_rot.shape[2]
    q_pos = q_pos.to(pos.device).reshape(-1, T).expand(B, T)
    out = torch.empty_like(q_rot)
    for r0 in range(0, T, rows):
        r1 = min(T, r0 + rows)
        w = torch.matmul(q_rot[:, :, r0:r1].contiguous(), Kt) * scale
        keep = pos[:, None, :] <= q_pos[:, r0:r1, None]       # [B, rows, L]
        if key_keep is not None:
            keep = keep & (key_keep[:, None, :] != 0)
        w = w.masked_fill(~keep[:, None], float("-inf"))
        p = F.softmax(w, dim=-1, dtype=torch.float32).to(q_rot.dtype)
        out[:, :, r0:r1] = torch.matmul(torch.nan_to_num(p), V)
    return out


def _keep_from_mask(mask, B, T):
    """Keep flags [B, T] (1 = attend) of the keys of the current call, from
    the HF attention mask handed to the attention module (4-D [B, 1, q, L]:
    additive float, 0 = attend, or bool, True = attend; or 2-D [B, L]).  The
    last query row covers every key of the call (causality lets it see
    them), and the call's keys are the last T columns.  None when the mask
    does not have that form."""
    if mask is None:
        return None
    row = mask[:, 0, -1, :] if mask.dim() == 4 else mask if mask.dim() == 2 else None
    if row is None or row.shape[0] != B or row.shape[-1] < T:
        return None
    row = row[:, -T:]
    if row.dtype == torch.bool:
        return row.to(torch.uint8)
    if row.is_floating_point():
        return (row == 0).to(torch.uint8)
    return (row != 0).to(torch.uint8)


def _cache_for(module, num_kv, head_dim, dtype, device, opts):
    cache = getattr(module, "_spectral_cache", None)
    if not isinstance(cache, SpectralCache) or cache.head_dim != head_dim or cache.device != device:
        cache = SpectralCache(num_heads=num_kv, head_dim=head_dim, block_size=opts["block_size"],
                              k_rank_keys=opts["k_rank_keys"], k_rank_values=opts["k_rank_values"],
                              hot_buffer_size=opts["hot_buffer_size"], device=device, dtype=torch.float16,
                              debug_logging=opts["debug_logging"],
                              use_attention_weighted_svd=opts["use_attention_weighted_svd"],
                              landmark_count=opts["landmark_count"],
                              quant_granularity=opts.get("quant_granularity", "per_head"))
        module._spectral_cache = cache
    return cache


def _attend(self, hidden_states, cos_cur, sin_cur, position_ids, attention_mask, opts, rope_mode):
    cfg = self.config
    Hq, Hkv = cfg.num_attention_heads, cfg.num_key_value_heads
    D = getattr(self, "head_dim", None) or cfg.hidden_size // Hq
    B, T, _ = hidden_states.shape
    q = self.q_proj(hidden_states).view(B, T, Hq, D).transpose(1, 2)
    k = self.k_proj(hidden_states).view(B, T, Hkv, D).transpose(1, 2)
    v = self.v_proj(hidden_states).view(B, T, Hkv, D).transpose(1, 2)
    cache = _cache_for(self, Hkv, D, hidden_states.dtype, hidden_states.device, opts)
    tab = _model_rope(self, D)
    if cos_cur is None:
        cur = position_ids
        if cur is None:
            start = cache.current_position
            cur = torch.arange(start, start + T, device=hidden_states.device)[None].expand(B, T)
        cos_all, sin_all = tab.get(cache.current_position + T + 1, hidden_states.device)
        cos_cur, sin_cur = cos_all[cur], sin_all[cur]
    q_rot = _rotate_queries(q, cos_cur, sin_cur)
    # Padding of a batched prompt (left padding): the HF mask of a
    # multi-sequence call marks the pad keys.  The cache keeps their flags,
    # and pad tokens get positions that continue backwards from the first
    # real token, so every sequence's real tokens are contiguous from the
    # position the model gave its first real token.
    # Only multi-token calls are inspected (one host read of the mask, like
    # the position read of a prefill); decode steps read nothing.
    keep_new = _keep_from_mask(attention_mask, B, T) if B > 1 and T > 1 else None
    if keep_new is not None and not bool((keep_new == 0).any()):
        keep_new = None
    store_pos = position_ids
    if keep_new is not None and position_ids is not None:
        store_pos = position_ids[:, -1:] - torch.arange(T - 1, -1, -1, device=position_ids.device)
    if T > 1:   # room for the prompt and the decode steps after it: those then allocate nothing
        cache.reserve(cache.current_position + T + opts.get("reserve_tokens", 4096), batch_size=B)
    cache.append(k, v, store_pos)                          # pre-RoPE K (integration.py:618-624)
    if keep_new is not None:
        cache.record_key_mask(keep_new, cache.total_tokens - T)
    cos_tab, sin_tab = tab.get(cache.current_position + 1, hidden_states.device)
    scale = getattr(self, "scaling", None) or 1.0 / math.sqrt(D)
    key_keep = cache.key_mask_view()
    if T == 1 and opts["use_spectral_attention"]:
        qpos = position_ids[:, -1] if position_ids is not None else cache.current_position - 1
        out = run_decode(q_rot, cache, cos_tab, sin_tab, qpos, key_keep, scale, rope_mode, halves_equal=True)
    elif opts["use_spectral_attention"] and prefill_supported(cache, Hq) and key_keep is None:
        qp = store_pos if store_pos is not None else \
            torch.arange(cache.current_position - T, cache.current_position, device=q_rot.device)[None]
        out = run_prefill(q_rot, cache, cos_tab, sin_tab, qp, scale)
    else:
        qp = store_pos if store_pos is not None else \
            torch.arange(cache.current_position - T, cache.current_position, device=q_rot.device)[None]
        out = _dense_prefill(q_rot, cache, cos_tab, sin_tab, Hq // Hkv, key_keep, scale, qp)
    out = out.to(hidden_states.dtype).transpose(1, 2).reshape(B, T, Hq * D)
    return self.o_proj(out), cache


def _options(block_size, k_rank_keys, k_rank_values, hot_buffer_size, use_spectral_attention, debug_logging,
             use_attention_weighted_svd, landmark_count, quant_granularity="per_head"):
    return dict(block_size=block_size, k_rank_keys=k_rank_keys, k_rank_values=k_rank_values,
                hot_buffer_size=hot_buffer_size, use_spectral_attention=use_spectral_attention,
                debug_logging=debug_logging, use_attention_weighted_svd=use_attention_weighted_svd,
                landmark_count=landmark_count, quant_granularity=quant_granularity)


def create_spectral_forward(original_forward, block_size=512, k_rank_keys=16, k_rank_values=32,
                            hot_buffer_size=64, use_spectral_attention=True, debug_logging=False,
                            use_attention_weighted_svd=False, landmark_count=0, rope_mode=None,
                            quant_granularity="per_head"):
    """Forward for an HF-style attention module (integration.py:43-425).
    Accepts both the transformers 5.x signature (position_embeddings) and
    the older one (position_ids, past_key_value)."""
    opts = _options(block_size, k_rank_keys, k_rank_values, hot_buffer_size, use_spectral_attention,
                    debug_logging, use_attention_weighted_svd, landmark_count, quant_granularity)
    mode = _lib.SC_ROPE_DISTANCE if rope_mode is None else rope_mode   # reference HF path: distance (:283)

    def spectral_forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                         past_key_values=None, **kwargs):
        position_ids = kwargs.get("position_ids")
        if position_ids is None and kwargs.get("cache_position") is not None:
            position_ids = kwargs["cache_position"][None].expand(hidden_states.shape[0], -1)
        cos_cur = sin_cur = None
        if position_embeddings is not None:
            cos_cur, sin_cur = position_embeddings
        out, cache = _attend(self, hidden_states, cos_cur, sin_cur, position_ids, attention_mask, opts, mode)
        return out, None

    return spectral_forward


def create_spectral_forward_inference(block_size=512, k_rank_keys=16, k_rank_values=32, hot_buffer_size=64,
                                      use_spectral_attention=True, debug_logging=False, use_triton_kernel=True,
                                      use_attention_weighted_svd=False, landmark_count=0):
    """Unsloth-signature decode function (integration.py:481-725):
    (self, hidden_states, past_key_value, position_ids, do_prefill, attention_mask)
    -> (attn_output, cache).  use_triton_kernel selects the absolute-RoPE
    path (the reference's Triton-module branch), otherwise distance RoPE."""
    opts = _options(block_size, k_rank_keys, k_rank_values, hot_buffer_size, use_spectral_attention,
                    debug_logging, use_attention_weighted_svd, landmark_count)
    mode = _lib.SC_ROPE_ABSOLUTE if use_triton_kernel else _lib.SC_ROPE_DISTANCE

    def spectral_forward_inference(self, hidden_states, past_key_value, position_ids, do_prefill=False,
                                   attention_mask=None):
        if isinstance(past_key_value, SpectralCache):
            self._spectral_cache = past_key_value
        out, cache = _attend(self, hidden_states, None, None, position_ids, attention_mask, opts, mode)
        return out, cache

    return spectral_forward_inference


def patch_unsloth_attention(model, block_size: int = 512, k_rank_keys: int = 16, k_rank_values: int = 32,
                            hot_buffer_size: int = 64, use_spectral_attention: bool = True, verbose: bool = True,
                            debug_logging: bool = False, use_triton_kernel: bool = True,
                            use_attention_weighted_svd: bool = False, landmark_count: int = 0,
                            quant_granularity: str = "per_head"):
    """Patches every ``model.model.layers[i].self_attn`` (integration.py:728-889).
    The decode path uses the absolute-RoPE kernel when ``use_triton_kernel``
    (the reference's default branch), distance RoPE otherwise."""
    _lib.load()
    rotary = getattr(getattr(model, "model", model), "rotary_emb", None)
    mode = _lib.SC_ROPE_ABSOLUTE if use_triton_kernel else _lib.SC_ROPE_DISTANCE
    n = 0
    for layer in model.model.layers:
        attn = getattr(layer, "self_attn", None)
        if attn is None:
            continue
        fwd = create_spectral_forward(attn.forward, block_size, k_rank_keys, k_rank_values, hot_buffer_size,
                                      use_spectral_attention, debug_logging, use_attention_weighted_svd,
                                      landmark_count, rope_mode=mode, quant_granularity=quant_granularity)
        attn.forward = fwd.__get__(attn, type(attn))
        attn._spectral_rope = _RopeTable(rotary, getattr(attn, "head_dim", None) or
                                         model.config.hidden_size // model.config.num_attention_heads,
                                         getattr(model.config, "rope_theta", 10000.0))
        attn._spectral_cache = None
        n += 1
    try:
        import unsloth.models.llama as llama_module  # noqa: F401
        llama_module.LlamaAttention_fast_forward_inference = create_spectral_forward_inference(
            block_size, k_rank_keys, k_rank_values, hot_buffer_size, use_spectral_attention, debug_logging,
            use_triton_kernel, use_attention_weighted_svd, landmark_count)
        if hasattr(llama_module, "_LlamaModel_fast_forward_inference"):
            llama_module.LlamaModel_fast_forward_inference = llama_module._LlamaModel_fast_forward_inference(
                attention_fast_forward_inference=llama_module.LlamaAttention_fast_forward_inference)
    except Exception as e:  # unsloth absent: the HF-style forward covers decode
        if verbose:
            print(f"(unsloth fast path not patched: {e.__class__.__name__}; HF-style forward in use)")
    if verbose:
        print(f"Patched {n} attention layers with SpectralCache (HIP)")
        print(f"   Config: block_size={block_size}, k_K={k_rank_keys}, k_V={k_rank_values}")
    return model


def reset_spectral_caches(model):
    """Drops every layer's cache (start of a new generation)."""
    for layer in model.model.layers:
        if hasattr(layer, "self_attn"):
            layer.self_attn._spectral_cache = None


def get_cache_stats(model):
    """integration.py:892-938"""
    total_tokens = total_blocks = orig = comp = 0
    per_layer = []
    for i, layer in enumerate(model.model.layers):
        cache = getattr(getattr(layer, "self_attn", None), "_spectral_cache", None)
        if isinstance(cache, SpectralCache):
            s = cache.get_memory_stats()
            total_tokens += s["total_tokens"]
            total_blocks += s["num_blocks"]
            orig += s["original_bytes"]
            comp += s["compressed_bytes"]
            per_layer.append({"layer_idx": i, "tokens": s["total_tokens"], "blocks": s["num_blocks"],
                              "compression": s["compression_ratio"]})
    return {"total_tokens": total_tokens, "total_blocks": total_blocks, "total_original_bytes": orig,
            "total_compressed_bytes": comp, "compression_ratio": orig / comp if comp > 0 else 1.0,
            "layers_with_cache": len(per_layer), "per_layer_stats": per_layer}


class CapturedDecode:
    """One-token decode steps of a patched model replayed from a HIP graph.

    The reference issues every decode step from Python (integration.py:596-659
    per layer); at batch 1 that host work, not the GPU, sets the token rate.
    Here one step of the whole model (every layer's append, spectral decode
    attention, projections and MLP) is captured once with
    ``torch.cuda.CUDAGraph`` and replayed for the following steps.  That is
    valid because the append and decode kernels take positions, tail lengths
    and block counts from the device counters; the only host-side launch
    arguments that change from step to step are the decode grid's extents,
    so each cache's tail grid is pinned for the segment (``steps`` tokens:
    workgroups past the device's tail length write neutral records) and the
    host mirror of the counters is advanced by the replays.

    Usage, after the prompt has been run through the patched model::

        dec = CapturedDecode(model, steps)
        for i in range(steps):
            logits = dec.step(token, position)   # [B, vocab]
            token, position = logits.argmax(-1), position + 1

    The first ``step`` runs eagerly (it also sizes the workspaces); the
    second captures; later ones replay.  ``token`` ([B] or [B, 1]) and
    ``position`` ([B, 1]) are device tensors; the returned logits of a replay
    live in the graph's static output, valid until the next ``step``.  The
    segment must not cross a block boundary (no compression inside it: every
    cache's tail length plus ``steps`` stays below ``block_size``), and the
    caches must hold room for it (``reserve``, as the prompt call does).
    ``close()`` (or the last step) unpins the grids."""

    def __init__(self, model, steps: int):
        self.model = model
        self.steps = int(steps)
        self.left = self.steps
        self.modules = [m for m in model.modules() if isinstance(getattr(m, "_spectral_cache", None), SpectralCache)]
        if not self.modules:
            raise ValueError("no spectral caches yet: run the prompt through the patched model first")
        self.caches = [m._spectral_cache for m in self.modules]
        for c in self.caches:
            if c._B is None:
                raise ValueError("empty spectral cache")
            if c._tail_len + self.steps >= c.block_size:
                raise ValueError(f"{self.steps} steps from a tail of {c._tail_len} cross a block boundary "
                                 f"({c.block_size}): split the segment at the compression")
            if c._tail_len + self.steps > c._tail_cap:
                raise ValueError("the tail ring has no room for the segment: reserve() first")
        for m, c in zip(self.modules, self.caches):
            tab = getattr(m, "_spectral_rope", None)
            if tab is not None:  # the tables must not be rebuilt inside the graph
                tab.get(c.current_position + self.steps + 2, c.device)
            c._grid_tail = c._tail_len + self.steps
        self.graph = None
        self.tok = self.pos = self.logits = None
        # A prepared 4-D mask is passed through by transformers as is, so no
        # mask is built inside the graph (building one copies a host scalar
        # to the device, which a capture refuses); the patched attention does
        # not read the mask of a one-token step (the cache keeps the prompt's
        # key flags).
        self.mask = None

    def _forward(self, token, position):
        if self.mask is None or self.mask.shape[0] != token.shape[0]:
            dtype = next(self.model.parameters()).dtype
            self.mask = torch.zeros(token.shape[0], 1, 1, 1, dtype=dtype, device=token.device)
        out = self.model(input_ids=token, position_ids=position, attention_mask=self.mask, use_cache=False,
                         logits_to_keep=1)
        return out.logits[:, -1]

    def _advance(self, n):
        for c in self.caches:
            c.total_tokens += n
            c.current_position += n
            c._tail_len += n

    @torch.no_grad()
    def step(self, token, position):
        if self.left <= 0:
            raise RuntimeError("the captured segment is used up")
        token = token.reshape(-1, 1)
        if self.left == self.steps:  # warm-up: eager, with the pinned grids
            logits = self._forward(token, position)
        else:
            if self.graph is None:
                self.tok = token.clone()
                self.pos = position.clone()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self.logits = self._forward(self.tok, self.pos)
                self._advance(-1)  # the capture ran the host side of a step, not its kernels
                self.graph = g
            self.tok.copy_(token)
            self.pos.copy_(position)
            self.graph.replay()
            self._advance(1)
            logits = self.logits
        self.left -= 1
        if self.left == 0:
            self.close()
        return logits

    def close(self):
        for c in self.caches:
            c._grid_tail = None
        self.left = 0
