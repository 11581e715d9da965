"""Spectral attention entry points (distance-RoPE path) and tensor helpers.

API of unsloth_spectral/spectral_attention.py:
  repeat_kv :38-47, repeat_kv_spectral :50-77, apply_rope :80-114,
  spectral_attention_forward :117-349, validate_spectral_attention :352-414.
``spectral_attention_forward`` runs the fused HIP decode kernel with the
reference's distance alignment: cold keys are rotated by d = max(q - p, 0)
(:192-219) using the first half of cos/sin for both halves; tail keys are
rotated at their absolute positions (:245-266).
"""
import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import _lib
from ._decode import run_decode
from .spectral_cache import SpectralBlock, SpectralCache  # noqa: F401  (re-export like the reference)


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, H_kv, T, D] -> [B, H_kv*n_rep, T, D] (query head h reads KV head h // n_rep)."""
    if n_rep == 1:
        return hidden_states
    b, h, t, d = hidden_states.shape
    return hidden_states[:, :, None].expand(b, h, n_rep, t, d).reshape(b, h * n_rep, t, d)


def repeat_kv_spectral(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[H_kv, ...] -> [H_kv*n_rep, ...] for coefficient / basis tensors."""
    if n_rep == 1:
        return x
    x = x.unsqueeze(1)
    sizes = list(x.shape)
    sizes[1] = n_rep
    return x.expand(*sizes).reshape(-1, *x.shape[2:])


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate (x[:D/2], x[D/2:]) pairs using the first half of cos/sin for both halves."""
    d = x.shape[-1]
    x1, x2 = x[..., :d // 2], x[..., d // 2:]
    c, s = cos[..., :d // 2], sin[..., :d // 2]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def spectral_attention_forward(
    Q: torch.Tensor,
    cache: SpectralCache,
    cos: torch.Tensor,
    sin: torch.Tensor,
    query_position,
    attention_mask: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Decode attention over the spectral cache, distance-RoPE alignment.

    Q [B, H_q, 1, D] post-RoPE; cos/sin [max_len, D]; query_position int or
    int tensor [B].  Returns [B, H_q, 1, D] in Q's dtype."""
    return run_decode(Q, cache, cos, sin, query_position, attention_mask, scale, _lib.SC_ROPE_DISTANCE)


def validate_spectral_attention(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cache: SpectralCache,
    rtol: float = 1e-2,
    atol: float = 1e-2,
    cos: Optional[torch.Tensor] = None,
    sin: Optional[torch.Tensor] = None,
    query_position: Optional[int] = None,
) -> Tuple[bool, dict]:
    """Spectral attention vs dense attention on the full K, V (:352-414).

    The reference calls spectral_attention_forward without cos/sin
    (:387, a TypeError); here, without tables both sides run unrotated
    (K, V and Q as given), with tables the dense side rotates K at its
    absolute positions and the spectral side uses the distance path."""
    B, H, _, D = Q.shape
    scale = 1.0 / math.sqrt(D)
    n_rep = H // K.shape[1]
    Kd = K
    if cos is not None:
        pos = cache.get_all_positions()
        Kd = apply_rope(K, cos[pos][None, None], sin[pos][None, None])
    scores_ref = torch.matmul(Q.float(), repeat_kv(Kd, n_rep).float().transpose(-2, -1)) * scale
    attn_ref = F.softmax(scores_ref, dim=-1)
    output_ref = torch.matmul(attn_ref, repeat_kv(V, n_rep).float()).to(Q.dtype)
    if cos is None:
        output = run_decode(Q, cache, None, None, 0, None, scale, _lib.SC_ROPE_NONE)
    else:
        qp = query_position if query_position is not None else cache.current_position - 1
        output = spectral_attention_forward(Q, cache, cos, sin, qp, scale=scale)
    abs_err = (output_ref.float() - output.float()).abs().max().item()
    rel_err = abs_err / (output_ref.float().abs().max().item() + 1e-8)
    mean_abs = (output_ref.float() - output.float()).abs().mean().item()
    K_recon, _ = cache.get_kv()
    if cos is not None:
        K_recon = apply_rope(K_recon, cos[pos][None, None], sin[pos][None, None])
    scores_sp = torch.matmul(Q.float(), repeat_kv(K_recon, n_rep).float().transpose(-2, -1)) * scale
    corr = torch.corrcoef(torch.stack([scores_ref.flatten(), scores_sp.flatten()]))[0, 1].item()
    ok = (abs_err < atol) or (rel_err < rtol)
    return ok, {"max_abs_error": abs_err, "max_rel_error": rel_err, "mean_abs_error": mean_abs,
                "attention_correlation": corr, "is_valid": ok}
