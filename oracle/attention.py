"""Compressed-space decode attention, restated from the reference (test infrastructure).

One sequence at a time (the reference cache is batch-1:
unsloth_spectral/spectral_cache.py:346); a batch of B sequences is B
independent calls.

* ``spectral_attention_forward`` -- distance-RoPE path,
  unsloth_spectral/spectral_attention.py:117-349 (cold alignment
  ``apply_rope(Q, cos[d], -sin[d])`` with d = clamp(q - p, 0), :192-219;
  ``apply_rope`` uses the first half of cos/sin for both halves, :80-114).
* ``spectral_attention_decode`` -- absolute-RoPE path,
  unsloth_spectral/kernels/spectral_attention.py:684-857 (cold score
  :375-453 with ``_apply_inverse_rope`` at the key's absolute position,
  :340-372; values :544-601).
* ``closed_form64`` -- float64 dense softmax attention over the
  dequantised reconstructed keys, each rotated by the reference's angle
  (absolute: p; distance: clamp(q - p, 0) for cold keys, p for the tail).

FP16 cast points kept from the reference (model dtype = float16):
  cold score   fp16(sum_k (fp32(Q_aligned) . B_k) * C_k)      spectral_attention.py:232-238
  tail score   fp16(Q . RoPE_p(K_tail))  (fp16 elementwise RoPE)  :258-273
  logits       fp16(fp16_scores * scale)                        :280-281
  probs        fp16(softmax_fp32(logits))                       :290
  cold value   fp16((P . C_V) . B_V) in fp32                    :322-328
  tail value   fp16(P_tail . V_tail)                            :343
  output       FP16 running sum over the parts                  :347
Elementwise FP16 arithmetic is evaluated like torch on the CPU: each op in
float32, rounded to float16.
"""
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

f16 = np.float16
f32 = np.float32


@dataclass
class ColdBlock:
    """One compressed block of one sequence (spectral_cache.py:20-46), with
    explicit INT8 codes.  ``scale_*`` is [H] (per head) or [H, T] (per row)."""
    codes_k: np.ndarray    # int8 [H, T, kK]
    scale_k: np.ndarray    # f32  [H] or [H, T]
    basis_k: np.ndarray    # f16  [H, kK, D]
    codes_v: np.ndarray    # int8 [H, T, kV]
    scale_v: np.ndarray
    basis_v: np.ndarray    # f16  [H, kV, D]
    start: int

    @property
    def T(self):
        return self.codes_k.shape[1]

    @staticmethod
    def _deq(codes, scale):
        s = np.asarray(scale, f32)
        s = s.reshape(s.shape + (1,) * (codes.ndim - s.ndim))
        return (codes.astype(f32) * s).astype(f32)

    def coeffs_k(self):
        """The reference's stored coefficients: fp16(round(x/s)*s), :404."""
        return self._deq(self.codes_k, self.scale_k).astype(f16)

    def coeffs_v(self):
        return self._deq(self.codes_v, self.scale_v).astype(f16)


@dataclass
class TierState:
    """Cold blocks + FP16 tail of one sequence (pre-RoPE keys)."""
    blocks: List[ColdBlock] = field(default_factory=list)
    tail_k: Optional[np.ndarray] = None   # f16 [H, Tt, D]
    tail_v: Optional[np.ndarray] = None
    tail_pos: Optional[np.ndarray] = None  # int [Tt]

    @property
    def num_heads(self):
        if self.blocks:
            return self.blocks[0].codes_k.shape[0]
        return self.tail_k.shape[0]

    @property
    def tail_len(self):
        return 0 if self.tail_k is None else self.tail_k.shape[1]

    def total_tokens(self):
        return sum(b.T for b in self.blocks) + self.tail_len

    def positions(self):
        """get_all_positions, spectral_cache.py:529-555."""
        parts = [np.arange(b.start, b.start + b.T) for b in self.blocks]
        if self.tail_len:
            parts.append(np.asarray(self.tail_pos).reshape(-1))
        return np.concatenate(parts) if parts else np.zeros(0, np.int64)

    def get_kv(self):
        """spectral_cache.py:557-612 -- fp16 reconstruction C.B per block
        (torch.bmm on fp16 operands), then the tail."""
        ks, vs = [], []
        for b in self.blocks:
            ks.append(np.matmul(b.coeffs_k().astype(f32), b.basis_k.astype(f32)).astype(f16))
            vs.append(np.matmul(b.coeffs_v().astype(f32), b.basis_v.astype(f32)).astype(f16))
        if self.tail_len:
            ks.append(self.tail_k)
            vs.append(self.tail_v)
        return np.concatenate(ks, axis=1), np.concatenate(vs, axis=1)


def _h(x):
    return np.asarray(x, f16)


def _rope_first_half(x, c, s):
    """spectral_attention.py:80-114 ``apply_rope`` (fp16 elementwise)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c1, s1 = c[..., :half], s[..., :half]
    out1 = _h(_h(x1 * c1) - _h(x2 * s1))
    out2 = _h(_h(x2 * c1) + _h(x1 * s1))
    return np.concatenate([out1, out2], axis=-1)


def _rope_halves(x, c, s):
    """kernels/spectral_attention.py:340-366 ``_apply_rope`` (fp16 elementwise)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2 = c[..., :half], c[..., half:]
    s1, s2 = s[..., :half], s[..., half:]
    out1 = _h(_h(x1 * c1) - _h(x2 * s1))
    out2 = _h(_h(x2 * c2) + _h(x1 * s2))
    return np.concatenate([out1, out2], axis=-1)


def _softmax32(logits16, mask):
    x = logits16.astype(f32)
    if mask is not None:
        x = np.where(np.asarray(mask) == 0, -np.inf, x)
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return (e / e.sum(axis=-1, keepdims=True)).astype(f32)


def _decode(Q, state, cos, sin, q, scale, mask, mode):
    Q = _h(Q)
    Hq, D = Q.shape
    Hkv = state.num_heads
    nrep = Hq // Hkv
    cos = _h(cos)
    sin = _h(sin)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    Qb = Q[:, None, :]                                     # [Hq, 1, D]
    parts = []
    for blk in state.blocks:
        kp = np.arange(blk.start, blk.start + blk.T)
        if mode == "distance":
            d = np.maximum(q - kp, 0)                      # spectral_attention.py:198
            qa = _rope_first_half(Qb, cos[d][None], (-sin[d])[None])   # :203-219
        else:
            qa = _rope_halves(Qb, cos[kp][None], (-sin[kp])[None])    # kernels/...:411-425
        basis = np.repeat(blk.basis_k, nrep, axis=0).astype(f32)      # repeat_kv
        coeffs = np.repeat(blk.coeffs_k(), nrep, axis=0).astype(f32)
        lat = np.matmul(qa.astype(f32), basis.transpose(0, 2, 1))     # einsum fp32
        parts.append((lat * coeffs).sum(-1).astype(f16))              # fp16 cast
    if state.tail_len:
        pos = np.asarray(state.tail_pos).reshape(-1)
        if mode == "distance":
            krot = _rope_first_half(_h(state.tail_k), cos[pos][None], sin[pos][None])
        else:
            krot = _rope_halves(_h(state.tail_k), cos[pos][None], sin[pos][None])
        krep = np.repeat(krot, nrep, axis=0).astype(f32)              # [Hq, Tt, D]
        parts.append(np.einsum("hd,htd->ht", Q.astype(f32), krep).astype(f16))
    if not parts:
        raise ValueError("Empty cache - no keys available")
    scores16 = np.concatenate(parts, axis=-1)                         # [Hq, Ttot]
    logits16 = (scores16.astype(f32) * f32(scale)).astype(f16)
    P = _softmax32(logits16, mask).astype(f16)
    out = None
    off = 0
    for blk in state.blocks:
        pb = P[:, off:off + blk.T].astype(f32)
        off += blk.T
        cv = np.repeat(blk.coeffs_v(), nrep, axis=0).astype(f32)      # [Hq, T, kV]
        bv = np.repeat(blk.basis_v, nrep, axis=0).astype(f32)         # [Hq, kV, D]
        vl = np.einsum("ht,htk->hk", pb, cv)
        o = np.einsum("hk,hkd->hd", vl, bv).astype(f16)
        out = o if out is None else _h(out.astype(f32) + o.astype(f32))
    if state.tail_len:
        pt = P[:, off:off + state.tail_len].astype(f32)
        vrep = np.repeat(_h(state.tail_v), nrep, axis=0).astype(f32)
        o = np.einsum("ht,htd->hd", pt, vrep).astype(f16)
        out = o if out is None else _h(out.astype(f32) + o.astype(f32))
    return out, scores16, logits16


def spectral_attention_forward(Q, state, cos, sin, query_position, scale=None, mask=None):
    """Distance-RoPE decode for one sequence.  Q: [Hq, D] post-RoPE query.
    Returns (out fp16 [Hq, D], raw scores fp16 [Hq, T], logits fp16)."""
    return _decode(Q, state, cos, sin, int(query_position), scale, mask, "distance")


def spectral_attention_decode(Q, state, cos, sin, query_position, scale=None, mask=None):
    """Absolute-RoPE decode for one sequence (same returns)."""
    return _decode(Q, state, cos, sin, int(query_position), scale, mask, "absolute")


def rotation_angles(state, query_position, mode):
    """Angle-table row used for every cached key, in cache order."""
    pos = state.positions().astype(np.int64)
    ncold = sum(b.T for b in state.blocks)
    if mode == "distance":
        ang = pos.copy()
        ang[:ncold] = np.maximum(int(query_position) - pos[:ncold], 0)
        return ang
    return pos


def closed_form64(Q, state, cos, sin, query_position, scale=None, mask=None, mode="absolute"):
    """float64 dense attention over the reconstructed keys, each key rotated
    *itself* by R at its angle row (keys, not the query, are rotated).

    With R acting on (x1, x2) pairs as
      cold, absolute : (c1 x1 - s2 x2,  s1 x1 + c2 x2)   [from Q.R_{-p}]
      tail, absolute : (c1 x1 - s1 x2,  s2 x1 + c2 x2)   [_apply_rope]
      distance       : (c1 x1 - s1 x2,  s1 x1 + c1 x2)   [apply_rope]
    Returns (out f64 [Hq, D], logits f64 [Hq, T])."""
    Q = np.asarray(Q, np.float64)
    Hq, D = Q.shape
    half = D // 2
    Hkv = state.num_heads
    nrep = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    cos = np.asarray(cos, np.float64)
    sin = np.asarray(sin, np.float64)
    Ks, Vs, kinds = [], [], []
    for b in state.blocks:
        Ks.append(np.matmul(b.coeffs_k().astype(np.float64), b.basis_k.astype(np.float64)))
        Vs.append(np.matmul(b.coeffs_v().astype(np.float64), b.basis_v.astype(np.float64)))
        kinds.append(np.zeros(b.T, bool))
    if state.tail_len:
        Ks.append(np.asarray(state.tail_k, np.float64))
        Vs.append(np.asarray(state.tail_v, np.float64))
        kinds.append(np.ones(state.tail_len, bool))
    K = np.concatenate(Ks, axis=1)            # [Hkv, T, D]
    V = np.concatenate(Vs, axis=1)
    is_tail = np.concatenate(kinds)
    ang = rotation_angles(state, query_position, mode)
    c, s = cos[ang], sin[ang]                 # [T, D]
    c1, c2, s1, s2 = c[:, :half], c[:, half:], s[:, :half], s[:, half:]
    x1, x2 = K[..., :half], K[..., half:]
    if mode == "distance":
        y1 = c1 * x1 - s1 * x2
        y2 = s1 * x1 + c1 * x2
    else:
        tail = is_tail[:, None]
        sa = np.where(tail, s1, s2)
        sb = np.where(tail, s2, s1)
        y1 = c1 * x1 - sa * x2
        y2 = sb * x1 + c2 * x2
    Kr = np.concatenate([y1, y2], axis=-1)
    Kr = np.repeat(Kr, nrep, axis=0)
    Vr = np.repeat(V, nrep, axis=0)
    logits = np.einsum("hd,htd->ht", Q, Kr) * scale
    if mask is not None:
        logits = np.where(np.asarray(mask) == 0, -np.inf, logits)
    m = logits.max(axis=-1, keepdims=True)
    e = np.exp(logits - m)
    P = e / e.sum(axis=-1, keepdims=True)
    return np.einsum("ht,htd->hd", P, Vr), logits


def spectral_score_forward(Q, coeffs_k, basis_k, cos, sin, start_position):
    """Scores of one block, kernels/spectral_attention.py:375-453
    (spectral_score_forward_pytorch): Q [Hq, D] fp16 post-RoPE, coeffs_k
    fp16 [Hkv, T, k], basis_k fp16 [Hkv, k, D].  Q is inverse-rotated at each
    key's absolute position with fp16 elementwise arithmetic (:411-425,
    _apply_inverse_rope :340-372), projected on the repeated basis in fp32
    (:436-440), multiplied by the coefficients and summed in fp32 (:444-445),
    cast to fp16 (:446).  Returns fp16 [Hq, T]."""
    Q = _h(Q)
    Hq, D = Q.shape
    Hkv, T, k = coeffs_k.shape
    nrep = Hq // Hkv
    kp = np.arange(int(start_position), int(start_position) + T)
    cos, sin = _h(cos), _h(sin)
    qa = _rope_halves(Q[:, None, :], cos[kp][None], (-sin[kp])[None])        # [Hq, T, D] fp16
    basis = np.repeat(_h(basis_k), nrep, axis=0).astype(f32)                 # [Hq, k, D]
    coeffs = np.repeat(_h(coeffs_k), nrep, axis=0).astype(f32)               # [Hq, T, k]
    lat = np.matmul(qa.astype(f32), basis.transpose(0, 2, 1))               # [Hq, T, k]
    return (lat * coeffs).sum(-1).astype(f16)


def spectral_value_forward(attn, coeffs_v, basis_v):
    """Values of one block, kernels/spectral_attention.py:544-601
    (spectral_value_forward_pytorch): attn [Hq, T] in fp32 (:585), coeffs_v
    fp16 [Hkv, T, k], basis_v fp16 [Hkv, k, D]; v_lat = attn . C in fp32
    (:587), out = v_lat . B in fp32 (:593), cast to fp16 (:594).
    Returns fp16 [Hq, D]."""
    attn = np.asarray(attn, f32)
    Hq = attn.shape[0]
    nrep = Hq // coeffs_v.shape[0]
    cv = np.repeat(_h(coeffs_v), nrep, axis=0).astype(f32)
    bv = np.repeat(_h(basis_v), nrep, axis=0).astype(f32)
    vl = np.einsum("ht,htk->hk", attn, cv)
    return np.einsum("hk,hkd->hd", vl, bv).astype(f16)
