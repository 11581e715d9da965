"""Cold-block wire format on the GPU (sc_tier_pack / sc_tier_unpack through
SpectralCache.export_blocks / import_blocks / save / load): records carry
the tiers bit for bit, headers describe them, foreign records are refused,
and decode over restored tiers equals decode over the originals exactly."""
import numpy as np
import pytest
import torch

from gpu_helpers import cache_from_states, tables
from helpers import random_state, rope_tables

pytestmark = pytest.mark.gpu

TIER = ("codes_k", "codes_v", "scales_k", "scales_v", "minmax_k", "minmax_v", "vnorm", "basis_k", "basis_v")


def _states(per_row, seed, B=2, H=8, nblk=3, T=128, kK=16, kV=32, tail=40):
    rng = np.random.default_rng(seed)
    return [random_state(rng, H, 128, nblk, T, kK, kV, tail, per_row=per_row, start=1000 * b) for b in range(B)]


def _decode(cache, Q, cos, sin, q):
    from unsloth_spectral import _lib
    from unsloth_spectral._decode import run_decode
    out = run_decode(Q, cache, cos, sin, q, rope_mode=_lib.SC_ROPE_ABSOLUTE, split=1)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("per_row", [False, True])
def test_export_import_round_trip_is_bit_exact(per_row):
    from unsloth_spectral import SpectralCache, wire
    src = cache_from_states(_states(per_row, 1), block_size=128)
    rec = src.export_blocks(seq=1)
    rb = src.block_record_bytes()
    assert rec.numel() == 3 * rb and rec.data_ptr() % 16 == 0
    hs = wire.headers(rec.cpu())
    assert [h.start_position for h in hs] == src.block_start[1, :3].tolist()
    assert all((h.kv_heads, h.head_dim, h.block_size, h.k_keys, h.k_values, h.granularity) ==
               (8, 128, 128, 16, 32, int(per_row)) for h in hs)
    # into sequence 0 of an empty cache of the same geometry, from host memory
    dst = SpectralCache(8, 128, block_size=128, k_rank_keys=16, k_rank_values=32, batch_size=2, max_blocks=1,
                        quant_granularity="per_row" if per_row else "per_head")
    assert dst.import_blocks(rec.cpu(), seq=0) == 3
    assert dst.num_cold_blocks == 3 and dst.counters[0, 0].item() == 3 and dst.counters[1, 0].item() == 0
    for name in TIER:
        assert torch.equal(getattr(dst, name)[0, :, :3], getattr(src, name)[1, :, :3]), name
    assert torch.equal(dst.block_start[0, :3], src.block_start[1, :3])


def test_offload_and_restore_gives_identical_decode():
    """Evict two blocks of a sequence (zeroed in HBM), bring them back from
    their records: the decode output is bit-identical to before."""
    states = _states(True, 2)
    cache = cache_from_states(states, block_size=128)
    total = states[0].total_tokens()
    cos, sin = tables(*rope_tables(total + 2100, 128))
    Q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(3)).half().cuda()
    q = torch.tensor([total - 1, 1000 + total - 1], dtype=torch.int32, device="cuda")
    before = _decode(cache, Q, cos, sin, q)
    rec = cache.export_blocks(seq=1, first=1, count=2).cpu()   # offload to host
    for name in TIER:
        getattr(cache, name)[1, :, 1:3].zero_()
    assert not torch.equal(_decode(cache, Q, cos, sin, q), before)
    cache.import_blocks(rec, seq=1, first=1)
    assert torch.equal(_decode(cache, Q, cos, sin, q), before)


def test_foreign_or_damaged_records_are_refused():
    from unsloth_spectral import SpectralCache
    from unsloth_spectral._lib import SpectralHIPError
    src = cache_from_states(_states(False, 4), block_size=128)
    rec = src.export_blocks(seq=0).cpu()
    other = SpectralCache(8, 128, block_size=128, k_rank_keys=32, k_rank_values=32, batch_size=1, max_blocks=4)
    with pytest.raises(ValueError):          # record size differs: refused on the host
        other.import_blocks(rec)
    same = SpectralCache(8, 128, block_size=128, k_rank_keys=16, k_rank_values=32, batch_size=1, max_blocks=4)
    bad = rec.clone()
    rb = src.block_record_bytes()
    bad[rb] ^= 0xFF                           # second record: magic damaged
    with pytest.raises(SpectralHIPError):
        same.import_blocks(bad)
    assert not torch.any(same.codes_k[0, :, :3]) and not torch.any(same.basis_v[0, :, :3])  # nothing taken
    assert same.num_cold_blocks == 0 and same.counters[0, 0].item() == 0
    assert same.import_blocks(rec) == 3 and torch.equal(same.codes_k[0, :, :3], src.codes_k[0, :, :3])


def test_save_and_load(tmp_path):
    from unsloth_spectral import SpectralCache
    states = _states(True, 5)
    cache = cache_from_states(states, block_size=128)
    total = states[0].total_tokens()
    cos, sin = tables(*rope_tables(total + 2100, 128))
    Q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(6)).half().cuda()
    q = torch.tensor([total - 1, 1000 + total - 1], dtype=torch.int32, device="cuda")
    path = str(tmp_path / "cache.safetensors")
    cache.save(path)
    back = SpectralCache.load(path)
    assert (back.num_cold_blocks, back.hot_len, back.total_tokens) == (cache.num_cold_blocks, cache.hot_len,
                                                                      cache.total_tokens)
    assert torch.equal(back.counters, cache.counters)
    assert torch.equal(_decode(back, Q, cos, sin, q), _decode(cache, Q, cos, sin, q))
