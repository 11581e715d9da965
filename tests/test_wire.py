"""Block wire format on the host: the Python layout rule equals the
library's (sc_block_record_bytes needs no GPU), the header codec round
trips, and validation rejects foreign or damaged headers."""
import ctypes

import pytest

from unsloth_spectral import wire

GEOMS = [  # kv_heads, head_dim, block_size, k_keys, k_values, per_row
    (8, 128, 512, 16, 32, False),
    (8, 128, 512, 32, 32, True),
    (2, 64, 128, 16, 16, True),
    (1, 128, 64, 64, 16, False),
    (3, 64, 192, 20, 40, True),
]


def _desc(H, D, T, kk, kv, per_row):
    from unsloth_spectral import _lib
    from unsloth_spectral.spectral_cache import padded_rank
    d = _lib.ScTierDesc()
    d.batch, d.kv_heads, d.head_dim, d.block_size = 1, H, D, T
    d.k_keys, d.k_values, d.kp_keys, d.kp_values = kk, kv, padded_rank(kk), padded_rank(kv)
    d.granularity = _lib.SC_QUANT_PER_ROW if per_row else _lib.SC_QUANT_PER_HEAD
    return d


@pytest.mark.parametrize("geom", GEOMS)
def test_record_size_matches_library(geom):
    from unsloth_spectral import _lib
    from unsloth_spectral.spectral_cache import padded_rank
    H, D, T, kk, kv, per_row = geom
    n_lib = _lib.load().sc_block_record_bytes(ctypes.byref(_desc(*geom)))
    n_py = wire.record_bytes(H, D, T, padded_rank(kk), padded_rank(kv), per_row)
    assert n_lib == n_py and n_py % 16 == 0
    offs, size = wire.layout(H, D, T, padded_rank(kk), padded_rank(kv), per_row)
    assert offs[0] == wire.HEADER_BYTES and all(o % 16 == 0 for o in offs)
    # sections follow each other in order, each large enough for its kv_heads slices
    hb = wire.section_head_bytes(T, D, padded_rank(kk), padded_rank(kv), per_row)
    for s in range(len(offs) - 1):
        assert offs[s + 1] >= offs[s] + hb[s] * H * (2 if s == 6 else 1)
    assert size >= offs[-1] + hb[-1] * H


def test_record_size_at_the_benchmark_geometry():
    # 8 KV heads x 512 tokens, k = 32, per-row scales: codes 2 x 131072, scales
    # 2 x 16384, bases 2 x 65536, minmax 128, vnorm 32, header 64
    assert wire.record_bytes(8, 128, 512, 32, 32, True) == 64 + 2 * 131072 + 2 * 16384 + 2 * 65536 + 128 + 32


def test_header_round_trip_and_validation():
    offs, size = wire.layout(8, 128, 512, 32, 32, True)
    h = wire.BlockHeader(wire.MAGIC, wire.VERSION, wire.HEADER_BYTES, size, 8, 128, 512, 32, 32, 32, 32, 1, 0,
                         1536, offs)
    raw = h.pack()
    assert len(raw) == 64 and raw[:4] == b"SCB1"
    back = wire.BlockHeader.unpack(raw)
    assert back == h
    back.validate()
    assert [x.start_position for x in wire.headers(raw + bytes(size - 64))] == [1536]
    for field, value in (("magic", 0x12345678), ("version", 2), ("record_bytes", size + 16)):
        bad = wire.BlockHeader.unpack(raw)
        setattr(bad, field, value)
        with pytest.raises(ValueError):
            bad.validate()
    bad = wire.BlockHeader.unpack(raw)
    bad.offsets[3] += 16
    with pytest.raises(ValueError):
        bad.validate()
