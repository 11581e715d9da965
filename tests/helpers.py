"""Shared test data: RoPE tables, synthetic tier states, parity metrics."""
import numpy as np

from oracle.attention import ColdBlock, TierState
from oracle.quant import quantize_per_head, quantize_per_row


def rope_tables(length, dim, theta=1e6, dtype=np.float16):
    """HF-style tables: inv_freq = theta^(-2i/D), emb = cat(freqs, freqs),
    cos/sin evaluated in float32 then cast (MistralRotaryEmbedding)."""
    inv = (1.0 / (theta ** (np.arange(0, dim, 2, dtype=np.float32) / dim))).astype(np.float32)
    freqs = np.outer(np.arange(length, dtype=np.float32), inv).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(dtype), np.sin(emb).astype(dtype)


def orthonormal_rows(rng, k, d):
    q, _ = np.linalg.qr(rng.standard_normal((d, k)))
    return q.T.astype(np.float32)


def random_state(rng, H, D, nblk, T, kK, kV, tail, per_row=False, start=0, coeff_std=1.5,
                 tail_std=0.75, tail_pos=None, batched_qr=False):
    """A tier state for one sequence: cold blocks with quantised Gaussian
    coefficients and orthonormal fp16 bases, plus an fp16 tail.
    batched_qr draws the bases of all heads of a block with one stacked QR
    (faster for large geometries; a different random stream)."""
    blocks = []
    for j in range(nblk):
        out = []
        for k in (kK, kV):
            coeffs = (rng.standard_normal((H, T, k)) * coeff_std).astype(np.float32)
            coeffs *= np.exp(-np.arange(k) / 8.0).astype(np.float32)
            if per_row:
                codes, scale, _, _ = quantize_per_row(coeffs)
            else:
                codes, scale, _, _ = quantize_per_head(coeffs)
            if batched_qr:
                q, _ = np.linalg.qr(rng.standard_normal((H, D, k)))
                basis = q.transpose(0, 2, 1).astype(np.float16)
            else:
                basis = np.stack([orthonormal_rows(rng, k, D) for _ in range(H)]).astype(np.float16)
            out.append((codes, scale, basis))
        (ck, sk, bk), (cv, sv, bv) = out
        blocks.append(ColdBlock(ck, sk, bk, cv, sv, bv, start + j * T))
    tk = tv = tp = None
    if tail:
        tk = (rng.standard_normal((H, tail, D)) * tail_std).astype(np.float16)
        tv = (rng.standard_normal((H, tail, D)) * tail_std).astype(np.float16)
        tp = np.arange(start + nblk * T, start + nblk * T + tail) if tail_pos is None else np.asarray(tail_pos)
    return TierState(blocks, tk, tv, tp)


def stack_states(states):
    """Arrays for SpectralCache.from_tiers from per-sequence TierStates."""
    import torch
    B = len(states)
    blocks0 = states[0].blocks
    nb = len(blocks0)
    H = states[0].num_heads
    D = blocks0[0].basis_k.shape[-1] if nb else states[0].tail_k.shape[-1]
    out = {}
    if nb:
        T, kK = blocks0[0].codes_k.shape[1:]
        kV = blocks0[0].codes_v.shape[2]
        f = lambda attr: np.stack([np.stack([getattr(b, attr) for b in s.blocks], 1) for s in states])  # noqa
        out["codes_k"] = torch.from_numpy(f("codes_k"))
        out["codes_v"] = torch.from_numpy(f("codes_v"))
        out["scales_k"] = torch.from_numpy(f("scale_k").astype(np.float32))
        out["scales_v"] = torch.from_numpy(f("scale_v").astype(np.float32))
        out["basis_k"] = torch.from_numpy(f("basis_k"))
        out["basis_v"] = torch.from_numpy(f("basis_v"))
        out["block_start"] = torch.tensor([[b.start for b in s.blocks] for s in states])
    else:
        out["codes_k"] = torch.zeros(B, H, 0, 512, 16, dtype=torch.int8)
        out["codes_v"] = torch.zeros(B, H, 0, 512, 16, dtype=torch.int8)
        out["scales_k"] = torch.ones(B, H, 0)
        out["scales_v"] = torch.ones(B, H, 0)
        out["basis_k"] = torch.zeros(B, H, 0, 16, D, dtype=torch.float16)
        out["basis_v"] = torch.zeros(B, H, 0, 16, D, dtype=torch.float16)
        out["block_start"] = torch.zeros(B, 0, dtype=torch.int32)
    if states[0].tail_len:
        out["tail_k"] = torch.from_numpy(np.stack([s.tail_k for s in states]))
        out["tail_v"] = torch.from_numpy(np.stack([s.tail_v for s in states]))
        out["tail_pos"] = torch.from_numpy(np.stack([np.asarray(s.tail_pos) for s in states]).astype(np.int32))
    return out


def pearson(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    a = a - a.mean()
    b = b - b.mean()
    return float((a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum()))


def lowrank_plus_noise(rng, n_mat, rows, cols, unit_scale=True, decay=8.0, noise=0.01):
    """U diag(sigma) V^T + noise per matrix, sigma_i = exp(-i/decay), U, V the
    Q factors of Gaussian draws; unit_scale lifts the low-rank term to unit
    RMS (the literal variant is noise-dominated).  Returns fp16 [n, rows, cols]."""
    sig = np.exp(-np.arange(cols) / decay)
    lift = np.sqrt(rows * cols / np.sum(sig ** 2)) if unit_scale else 1.0
    out = np.empty((n_mat, rows, cols), np.float32)
    for i in range(n_mat):
        U, _ = np.linalg.qr(rng.standard_normal((rows, cols)))
        V, _ = np.linalg.qr(rng.standard_normal((cols, cols)))
        out[i] = (U * (sig * lift)) @ V.T + noise * rng.standard_normal((rows, cols))
    return out.astype(np.float16)
