"""Writes the small fixtures of tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

* quant_vectors.npz    -- inputs with exact .5 ties, expected per-head and
                          per-row codes/scales (closed form of
                          spectral_cache.py:481-516)
* rsvd_known_answer.json -- the reference self-test's seeded case
                          (rsvd.py:160-220) with its published answers
                          (PHASE2_RSVD_OPTIMIZATION.md:40-41) and a checksum
                          of the regenerated M
* decode_tiny.npz      -- a tiny tier state (H_kv=2, H_q=8, D=128, two
                          128-token blocks, k=16/32, 100-token tail, theta=1e6)
                          with float64 outputs of both RoPE modes computed by
                          transformers' apply_rotary_pos_emb + eager
                          attention on the reconstructed keys (independent of
                          the oracle's query-side formulation)
No file of the reference is imported or run.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from golden_io import save_decode_case  # noqa: E402
from helpers import random_state, rope_tables  # noqa: E402


def quant_vectors():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((3, 64, 16)) * 2).astype(np.float32)
    s = np.float32(1 / 16)
    x[0, 0, :11] = np.array([127.0, 0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5, 126.5, -126.5], np.float32) * s
    x[0, 1:] = np.clip(x[0, 1:], -126 * s, 126 * s)
    x[1] = 0.0
    x[2, 5] *= 50
    scale_h = np.maximum(np.abs(x).max(axis=(1, 2)), np.float32(1e-8)) / np.float32(127)
    codes_h = np.rint(x / scale_h[:, None, None]).astype(np.int8)
    scale_r = np.maximum(np.abs(x).max(axis=2), np.float32(1e-8)) / np.float32(127)
    codes_r = np.rint(x / scale_r[..., None]).astype(np.int8)
    assert codes_h[0, 0, :11].tolist() == [127, 0, 2, 2, 4, 0, -2, -2, -4, 126, -126]
    np.savez_compressed(os.path.join(HERE, "quant_vectors.npz"), x=x, codes_per_head=codes_h,
                        scales_per_head=scale_h.astype(np.float32), codes_per_row=codes_r,
                        scales_per_row=scale_r.astype(np.float32))


def rsvd_known_answer():
    import torch
    torch.manual_seed(42)
    M = torch.randn(8, 512, 16) @ torch.randn(8, 16, 128) + 0.1 * torch.randn(8, 512, 128)
    ka = {"seed": 42, "B": 8, "m": 512, "n": 128, "k": 16, "oversampling": 5, "n_iter": 2,
          "err_published": 0.022725, "s_abs_err_published": 0.000072,
          "source": "PHASE2_RSVD_OPTIMIZATION.md:40-41 (reference self-test rsvd.py:160-220)",
          "m_checksum": float(M.double().sum())}
    with open(os.path.join(HERE, "rsvd_known_answer.json"), "w") as f:
        json.dump(ka, f, indent=1)


def hf_dense64(Q, st, cos, sin, angles):
    import torch
    from transformers.models.mistral.modeling_mistral import apply_rotary_pos_emb
    K, V = st.get_kv()
    Kt = torch.from_numpy(K.astype(np.float64))[None]
    Vt = torch.from_numpy(V.astype(np.float64))[None]
    c = torch.from_numpy(cos[angles].astype(np.float64))[None]
    s = torch.from_numpy(sin[angles].astype(np.float64))[None]
    _, Kr = apply_rotary_pos_emb(Kt, Kt, c, s)
    rep = Q.shape[0] // K.shape[0]
    Qt = torch.from_numpy(Q.astype(np.float64))[None, :, None]
    p = torch.softmax((Qt @ Kr.repeat_interleave(rep, 1).transpose(-1, -2)) / np.sqrt(Q.shape[-1]), dim=-1)
    return (p @ Vt.repeat_interleave(rep, 1))[0, :, 0].numpy()


def decode_tiny():
    rng = np.random.default_rng(12)
    st = random_state(rng, 2, 128, 2, 128, 16, 32, 100)
    total = st.total_tokens()
    cos, sin = rope_tables(total + 8, 128)
    Q = rng.standard_normal((8, 128)).astype(np.float16)
    q = total - 1
    pos = st.positions()
    ang = pos.copy()
    ang[:256] = q - pos[:256]
    save_decode_case(os.path.join(HERE, "decode_tiny.npz"), Q, st, cos, sin, q,
                     out64_absolute=hf_dense64(Q, st, cos, sin, pos),
                     out64_distance=hf_dense64(Q, st, cos, sin, ang))


if __name__ == "__main__":
    quant_vectors()
    rsvd_known_answer()
    decode_tiny()
    print("fixtures written to", HERE)
