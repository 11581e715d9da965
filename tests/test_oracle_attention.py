"""Pins the decode-attention restatement (oracle/attention.py).

The FP16-faithful restatement follows the reference's structure (query
inverse-rotated per key, latent projection, fp16 casts); it must agree with
structurally different computations:
* ``closed_form64``: dense softmax attention in float64 over the
  reconstructed keys, each key rotated itself;
* transformers' own ``apply_rotary_pos_emb`` + eager attention for the
  absolute mode (keys at absolute positions) and for the distance mode
  (cold keys at q - p, tail keys at p).
A sign error in the rotation, a wrong angle index, a dropped tail or a
transposed basis fails these comparisons.
"""
import os

import numpy as np
import pytest

from helpers import pearson, random_state, rope_tables
from oracle.attention import closed_form64, spectral_attention_decode, spectral_attention_forward

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _case(seed=0, H=2, rep=4, D=128, nblk=2, T=128, kK=16, kV=32, tail=100, per_row=False, qscale=1.0):
    rng = np.random.default_rng(seed)
    st = random_state(rng, H, D, nblk, T, kK, kV, tail, per_row=per_row)
    total = st.total_tokens()
    cos, sin = rope_tables(total + 8, D)
    Q = (rng.standard_normal((H * rep, D)) * qscale).astype(np.float16)
    return st, cos, sin, Q, total


@pytest.mark.parametrize("mode", ["absolute", "distance"])
@pytest.mark.parametrize("per_row", [False, True])
def test_fp16_restatement_vs_closed_form(mode, per_row):
    st, cos, sin, Q, total = _case(seed=1, per_row=per_row)
    q = total - 1
    fn = spectral_attention_decode if mode == "absolute" else spectral_attention_forward
    out, scores16, logits16 = fn(Q, st, cos, sin, q)
    ref, lg = closed_form64(Q, st, cos, sin, q, mode=mode)
    err = np.abs(out.astype(np.float64) - ref).max()
    assert err < 2e-3 and err < 1e-2 * np.abs(ref).max(), err
    assert pearson(logits16, lg) > 0.9999


def _hf_dense(Q, st, cos, sin, angles, scale=None):
    torch = pytest.importorskip("torch")
    from transformers.models.mistral.modeling_mistral import apply_rotary_pos_emb
    K, V = st.get_kv()                                   # fp16 [Hkv, T, D]
    Kt = torch.from_numpy(K.astype(np.float64))[None]
    Vt = torch.from_numpy(V.astype(np.float64))[None]
    c = torch.from_numpy(cos[angles].astype(np.float64))[None]
    s = torch.from_numpy(sin[angles].astype(np.float64))[None]
    _, Kr = apply_rotary_pos_emb(Kt, Kt, c, s)
    Qt = torch.from_numpy(Q.astype(np.float64))[None, :, None]
    rep = Q.shape[0] // K.shape[0]
    Kr = Kr.repeat_interleave(rep, dim=1)
    Vr = Vt.repeat_interleave(rep, dim=1)
    scale = scale or 1 / np.sqrt(Q.shape[-1])
    p = torch.softmax((Qt @ Kr.transpose(-1, -2)) * scale, dim=-1)
    return (p @ Vr)[0, :, 0].numpy()


def test_absolute_mode_is_hf_dense_attention():
    st, cos, sin, Q, total = _case(seed=2)
    out, _, _ = spectral_attention_decode(Q, st, cos, sin, total - 1)
    ref = _hf_dense(Q, st, cos, sin, st.positions())
    assert np.abs(out.astype(np.float64) - ref).max() < 2e-3


def test_distance_mode_rotates_cold_keys_by_q_minus_p():
    st, cos, sin, Q, total = _case(seed=3)
    q = total - 1
    out, _, _ = spectral_attention_forward(Q, st, cos, sin, q)
    pos = st.positions()
    ncold = sum(b.T for b in st.blocks)
    ang = pos.copy()
    ang[:ncold] = q - pos[:ncold]
    ref = _hf_dense(Q, st, cos, sin, ang)
    assert np.abs(out.astype(np.float64) - ref).max() < 2e-3
    # and it is NOT dense attention at absolute positions (different math)
    ref_abs = _hf_dense(Q, st, cos, sin, pos)
    assert np.abs(ref - ref_abs).max() > 1e-2


def test_tail_only_cache_both_modes_equal_dense():
    st, cos, sin, Q, total = _case(seed=4, nblk=0, tail=77)
    ref = _hf_dense(Q, st, cos, sin, st.positions())
    for fn in (spectral_attention_decode, spectral_attention_forward):
        out, _, _ = fn(Q, st, cos, sin, total - 1)
        assert np.abs(out.astype(np.float64) - ref).max() < 2e-3


def test_mask_drops_keys():
    st, cos, sin, Q, total = _case(seed=5)
    rng = np.random.default_rng(6)
    mask = (rng.random((Q.shape[0], total)) > 0.3).astype(np.int64)
    out, _, _ = spectral_attention_decode(Q, st, cos, sin, total - 1, mask=mask)
    ref, _ = closed_form64(Q, st, cos, sin, total - 1, mask=mask)
    assert np.abs(out.astype(np.float64) - ref).max() < 2e-3
    ref_nomask, _ = closed_form64(Q, st, cos, sin, total - 1)
    assert np.abs(ref - ref_nomask).max() > 1e-2


def test_empty_cache_raises():
    from oracle.attention import TierState
    cos, sin = rope_tables(8, 128)
    with pytest.raises(ValueError):
        spectral_attention_decode(np.zeros((4, 128), np.float16), TierState([], np.zeros((1, 0, 128), np.float16),
                                                                            np.zeros((1, 0, 128), np.float16),
                                                                            np.zeros(0, int)), cos, sin, 0)


def test_golden_decode_tiny():
    path = os.path.join(GOLDEN, "decode_tiny.npz")
    if not os.path.exists(path):
        pytest.skip("fixture missing (run tests/golden/make_golden.py)")
    from golden_io import load_decode_case
    case = load_decode_case(path)
    for mode, fn in (("absolute", spectral_attention_decode), ("distance", spectral_attention_forward)):
        out, _, _ = fn(case["Q"], case["state"], case["cos"], case["sin"], case["q"])
        assert np.abs(out.astype(np.float64) - case[f"out64_{mode}"]).max() < 2e-3


def test_block_score_restatement_vs_closed_form():
    """spectral_score_forward: q . R_p(C_t B) in float64 with every key
    rotated itself at its absolute position p = start + t by the reference's
    _apply_rope halves (x1 c1 - x2 s1, x2 c2 + x1 s2), against the
    restatement that inverse-rotates the query instead.  Unequal table
    halves make a swapped half or a wrong sign fail."""
    from oracle.attention import spectral_score_forward
    rng = np.random.default_rng(70)
    Hkv, rep, T, k, D, start = 2, 4, 96, 16, 128, 300
    cos, sin = rope_tables(start + T + 4, D)
    cos = cos.copy()
    cos[:, D // 2:] = (cos[:, D // 2:].astype(np.float32) * 0.9).astype(np.float16)
    coeffs = (rng.standard_normal((Hkv, T, k)) * 0.8).astype(np.float16)
    basis = (rng.standard_normal((Hkv, k, D)) / np.sqrt(D)).astype(np.float16)
    Q = rng.standard_normal((Hkv * rep, D)).astype(np.float16)
    got = spectral_score_forward(Q, coeffs, basis, cos, sin, start).astype(np.float64)
    K = np.matmul(coeffs.astype(np.float64), basis.astype(np.float64))      # [Hkv, T, D]
    p = np.arange(start, start + T)
    c, s = cos[p].astype(np.float64), sin[p].astype(np.float64)
    h = D // 2
    x1, x2 = K[..., :h], K[..., h:]
    Kr = np.concatenate([x1 * c[:, :h] - x2 * s[:, :h], x2 * c[:, h:] + x1 * s[:, h:]], axis=-1)
    ref = np.einsum("hd,htd->ht", Q.astype(np.float64), np.repeat(Kr, rep, axis=0))
    assert np.abs(got - ref).max() <= 5e-3 * np.abs(ref).max()
    assert pearson(got, ref) > 0.99999


def test_block_value_restatement_vs_closed_form():
    """spectral_value_forward: float64 P . (C B) with the query head h using
    KV head h // rep (repeat_interleave), against the restatement's
    (P . C) . B in fp32."""
    from oracle.attention import spectral_value_forward
    rng = np.random.default_rng(71)
    Hkv, rep, T, k, D = 2, 4, 200, 32, 128
    coeffs = (rng.standard_normal((Hkv, T, k)) * 0.8).astype(np.float16)
    basis = (rng.standard_normal((Hkv, k, D)) / np.sqrt(D)).astype(np.float16)
    P = rng.random((Hkv * rep, T)).astype(np.float32)
    P /= P.sum(-1, keepdims=True)
    got = spectral_value_forward(P, coeffs, basis).astype(np.float64)
    V = np.matmul(coeffs.astype(np.float64), basis.astype(np.float64))
    ref = np.einsum("ht,htd->hd", P.astype(np.float64), np.repeat(V, rep, axis=0))
    assert np.abs(got - ref).max() <= 2e-3 * np.abs(ref).max() + 1e-6
    # head 5 reads KV head 1: using KV head 0 instead is far off
    wrong = P[5].astype(np.float64) @ V[0]
    assert np.abs(wrong - ref[5]).max() > 10 * np.abs(got[5] - ref[5]).max()
