"""Decode-path entry points of the kernels module (absolute-RoPE path).

API of unsloth_spectral/kernels/spectral_attention.py:
  TritonSpectralConfig :50-65, _apply_rope / _apply_inverse_rope :340-372,
  spectral_score_forward :375-541, spectral_value_forward :544-677,
  spectral_attention_decode :684-857.
The per-block Triton/PyTorch loops are replaced by the fused HIP kernel:
``spectral_attention_decode`` is one split-K launch + one combine launch for
every cold block and the FP16 tail of every sequence, with cold keys aligned
at their absolute positions (the reference's inverse RoPE of Q by p, :411-425)
and tail keys rotated by ``_apply_rope`` (:776).
"""
import math
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib
from .._decode import run_decode
from ..spectral_cache import SpectralCache


@dataclass
class TritonSpectralConfig:
    """Launch knobs of the reference's Triton kernels (:50-65).  The tile
    fields are accepted for API compatibility; the HIP kernel's tiling is
    fixed (16-token MFMA tiles, 64-token ranges, four wavefronts per
    workgroup) and nothing is logged per block.  ``split_blocks`` is this
    kernel's one launch knob: workgroups per cold block (0 = chosen from the
    grid size; fix it to get bit-identical results across batch sizes)."""
    BLOCK_T: int = 64
    BLOCK_K: int = 32
    BLOCK_D: int = 64
    num_warps: int = 4
    num_stages: int = 2
    enable_logging: bool = True
    split_blocks: int = 0

    def __post_init__(self):
        assert self.BLOCK_T >= 16, "BLOCK_T must be at least 16"
        assert self.BLOCK_K >= 8, "BLOCK_K must be at least 8"
        assert self.BLOCK_D >= 32, "BLOCK_D must be at least 32"


def _apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """(x1 c1 - x2 s1, x2 c2 + x1 s2) with halves of cos/sin (:340-366)."""
    d = x.shape[-1]
    x1, x2 = x[..., :d // 2], x[..., d // 2:]
    return torch.cat([x1 * cos[..., :d // 2] - x2 * sin[..., :d // 2],
                      x2 * cos[..., d // 2:] + x1 * sin[..., d // 2:]], dim=-1)


def _apply_inverse_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    return _apply_rope(x, cos, -sin)


def spectral_attention_decode(
    Q: torch.Tensor,
    cache: SpectralCache,
    cos: torch.Tensor,
    sin: torch.Tensor,
    query_position,
    attention_mask: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    config: Optional[TritonSpectralConfig] = None,
) -> torch.Tensor:
    """Decode attention over the spectral cache, absolute-RoPE alignment.
    Q [B, H_q, 1, D] post-RoPE -> [B, H_q, 1, D]."""
    return run_decode(Q, cache, cos, sin, query_position, attention_mask, scale, _lib.SC_ROPE_ABSOLUTE,
                      split=config.split_blocks if config is not None else 0)


def _one_block_cache(coeffs, basis, start_position, kind, D, B):
    """A one-block cache (B copies) holding `coeffs` [H, T, k] (reference fp16
    coefficients) as INT8 codes with scale = max|coeff|/127 per head."""
    H, T, k = coeffs.shape
    c = coeffs.float()
    absmax = torch.clamp(c.abs().amax(dim=(1, 2)), min=1e-8)
    scale = absmax / 127.0
    codes = torch.round(c / scale[:, None, None]).to(torch.int8)[None, :, None].expand(B, H, 1, T, k)
    sc = scale[None, :, None].expand(B, H, 1)
    bas = basis.to(torch.float16)[None, :, None].expand(B, H, 1, k, D)
    z_codes = torch.zeros(B, H, 1, T, 16, dtype=torch.int8, device=coeffs.device)
    z_basis = torch.zeros(B, H, 1, 16, D, dtype=torch.float16, device=coeffs.device)
    ones = torch.ones(B, H, 1, device=coeffs.device)
    start = torch.full((B, 1), int(start_position), device=coeffs.device)
    if kind == "K":
        return SpectralCache.from_tiers(codes, sc, bas, z_codes, ones, z_basis, start, block_size=T)
    return SpectralCache.from_tiers(z_codes, ones, z_basis, codes, sc, bas, start, block_size=T)


def spectral_score_forward(Q, coeffs_K, basis_K, cos, sin, start_position, query_position,
                           config: Optional[TritonSpectralConfig] = None, use_triton: bool = False):
    """Raw cold-block scores [B, H_q, 1, T_block] in Q's dtype (:375-541):
    Q . R_p(coeffs_K @ basis_K) with p = start_position + t.  Coefficients
    are held as INT8 codes (exact for coefficients produced by the
    reference quantiser, :481-516)."""
    B, Hq, _, D = Q.shape
    T = coeffs_K.shape[1]
    cache = _one_block_cache(coeffs_K, basis_K, start_position, "K", D, B)
    logits = torch.empty(B, Hq, T, dtype=torch.float32, device=Q.device)
    run_decode(Q, cache, cos, sin, query_position, None, 1.0, _lib.SC_ROPE_ABSOLUTE, logits=logits)
    return logits.to(Q.dtype).unsqueeze(2)


def spectral_value_forward(attn, coeffs_V, basis_V, D, config: Optional[TritonSpectralConfig] = None,
                           use_triton: bool = False):
    """(attn @ coeffs_V) @ basis_V per query head with GQA (:544-601), fp32
    accumulation, result in attn's dtype.  A small per-block helper outside
    the fused path (the fused kernel applies B_V once per block itself)."""
    B, Hq, _, T = attn.shape
    Hkv = coeffs_V.shape[0]
    n_rep = Hq // Hkv
    cv = coeffs_V.float().repeat_interleave(n_rep, dim=0)
    bv = basis_V.float().repeat_interleave(n_rep, dim=0)
    v_lat = torch.matmul(attn.float(), cv.unsqueeze(0))
    return torch.matmul(v_lat, bv.unsqueeze(0)).to(attn.dtype)


def spectral_attention_decode_pytorch(Q, cache, cos, sin, query_position, attention_mask=None, scale=None):
    """Same interface, distance path (reference :864-879 forwards there too)."""
    from ..spectral_attention import spectral_attention_forward
    return spectral_attention_forward(Q, cache, cos, sin, query_position, attention_mask, scale)
