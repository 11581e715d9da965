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


def _fp16_rows(t, D):
    """fp16, contiguous, 16-byte aligned rows (what the block kernels read)."""
    t = t.to(torch.float16)
    if not t.is_contiguous() or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def spectral_score_forward(Q, coeffs_K, basis_K, cos, sin, start_position, query_position,
                           config: Optional[TritonSpectralConfig] = None, use_triton: bool = False):
    """Raw cold-block scores [B, H_q, 1, T_block] (:375-541): Q aligned by
    the inverse RoPE at each key's absolute position start_position + t,
    projected on basis_K [H_kv, k, D] in fp32, times coeffs_K [H_kv, T, k]
    and summed in fp32, rounded to fp16 (sc_block_scores).  ``use_triton``
    selected the reference's Triton kernel; there is one HIP kernel here.
    ``query_position`` does not enter the absolute alignment (as in the
    reference)."""
    _lib.require_device(Q, "Q")
    B, Hq, _, D = Q.shape
    Hkv, T, k = coeffs_K.shape
    if basis_K.shape != (Hkv, k, D):
        raise ValueError(f"basis_K must be [{Hkv}, {k}, {D}], got {tuple(basis_K.shape)}")
    q = _fp16_rows(Q.reshape(B, Hq, D), D)
    ck = _fp16_rows(coeffs_K, D)
    bk = _fp16_rows(basis_K, D)
    c16 = cos.to(torch.float16).contiguous()
    s16 = sin.to(torch.float16).contiguous()
    scores = torch.empty(B, Hq, T, dtype=torch.float16, device=Q.device)
    lib = _lib.load()
    _lib.check(lib.sc_block_scores(_lib.ptr(q), q.stride(0), q.stride(1), B, Hq, _lib.ptr(ck), _lib.ptr(bk), Hkv,
                                   T, k, D, _lib.ptr(c16), _lib.ptr(s16), c16.stride(0),
                                   min(c16.shape[0], s16.shape[0]), int(start_position), _lib.ptr(scores),
                                   _lib.stream_of(Q)))
    return scores.to(Q.dtype).unsqueeze(2)


def spectral_value_forward(attn, coeffs_V, basis_V, D, config: Optional[TritonSpectralConfig] = None,
                           use_triton: bool = False):
    """(attn @ coeffs_V) @ basis_V per query head with GQA (:544-601):
    attn [B, H_q, 1, T] taken in fp32 as the reference does, both products
    summed in fp32, result [B, H_q, 1, D] in attn's dtype (sc_block_values).
    The fused decode kernel applies B_V once per block itself; this is the
    per-block helper of the reference's API."""
    _lib.require_device(attn, "attn")
    B, Hq, _, T = attn.shape
    Hkv, T2, k = coeffs_V.shape
    if T2 != T or basis_V.shape != (Hkv, k, D):
        raise ValueError(f"coeffs_V [{Hkv}, {T}, k] and basis_V [{Hkv}, k, {D}] expected, got "
                         f"{tuple(coeffs_V.shape)} and {tuple(basis_V.shape)}")
    a = attn.reshape(B, Hq, T).float()
    if a.stride(-1) != 1:
        a = a.contiguous()
    cv = _fp16_rows(coeffs_V, D)
    bv = _fp16_rows(basis_V, D)
    out = torch.empty(B, Hq, D, dtype=torch.float16, device=attn.device)
    lib = _lib.load()
    _lib.check(lib.sc_block_values(_lib.ptr(a), a.stride(0), a.stride(1), B, Hq, _lib.ptr(cv), _lib.ptr(bv), Hkv, T,
                                   k, D, _lib.ptr(out), _lib.stream_of(attn)))
    return out.to(attn.dtype).unsqueeze(2)


def spectral_attention_decode_pytorch(Q, cache, cos, sin, query_position, attention_mask=None, scale=None):
    """Same interface, distance path (reference :864-879 forwards there too)."""
    from ..spectral_attention import spectral_attention_forward
    return spectral_attention_forward(Q, cache, cos, sin, query_position, attention_mask, scale)
