"""Helpers shared by the GPU tests (device transfer, cache export)."""
import numpy as np
import torch

from helpers import stack_states
from oracle.attention import ColdBlock, TierState


def cache_from_states(states, block_size=None, tail_capacity=None):
    from unsloth_spectral import SpectralCache
    a = {k: v.cuda() for k, v in stack_states(states).items()}
    T = block_size or (states[0].blocks[0].T if states[0].blocks else 512)
    return SpectralCache.from_tiers(a["codes_k"], a["scales_k"], a["basis_k"], a["codes_v"], a["scales_v"],
                                    a["basis_v"], a["block_start"], a.get("tail_k"), a.get("tail_v"),
                                    a.get("tail_pos"), block_size=T, tail_capacity=tail_capacity)


def export_states(cache):
    """Per-sequence oracle TierStates holding exactly the GPU cache's tiers."""
    B = cache._B
    kK, kV, nb = cache.k_rank_keys, cache.k_rank_values, cache.num_cold_blocks
    per_row = cache.quant_granularity == "per_row"
    ck = cache.codes_k[:, :, :nb, :, :kK].cpu().numpy()
    cv = cache.codes_v[:, :, :nb, :kV, :].transpose(-1, -2).cpu().numpy()
    sk = cache.scales_k[:, :, :nb].cpu().numpy()
    sv = cache.scales_v[:, :, :nb].cpu().numpy()
    bk = cache.basis_k[:, :, :nb, :, :kK].transpose(-1, -2).cpu().numpy()
    bv = cache.basis_v[:, :, :nb, :, :kV].transpose(-1, -2).cpu().numpy()
    starts = cache.block_start[:, :nb].cpu().numpy()
    hk, hv, hp = cache.hot_K, cache.hot_V, cache.hot_position_ids
    out = []
    for b in range(B):
        blocks = [ColdBlock(ck[b, :, j], sk[b, :, j], bk[b, :, j], cv[b, :, j], sv[b, :, j], bv[b, :, j],
                            int(starts[b, j])) for j in range(nb)]
        if hk is not None:
            out.append(TierState(blocks, hk[b].cpu().numpy(), hv[b].cpu().numpy(), hp[b].cpu().numpy()))
        else:
            out.append(TierState(blocks, None, None, None))
    return out


def tables(cos, sin):
    return torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
