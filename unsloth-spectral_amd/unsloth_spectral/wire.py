"""Cold-block wire format: host-side view of the records that
``sc_tier_pack`` writes and ``sc_tier_unpack`` reads (layout: ScBlockHeader
in include/spectral_hip.h).

The reference has no serialised block (spectral_cache.py:20-46 keeps
SpectralBlock as tensors; :614-655 only counts bytes).  A record is a
64-byte little-endian header followed by eight 16-byte aligned sections:
codes_k, codes_v, scales_k, scales_v, basis_k, basis_v, minmax (K then V),
vnorm.  ``record_bytes`` restates the library's layout rule so a host can
size and walk a buffer of records without the GPU.
"""
import struct
from dataclasses import dataclass
from typing import List

MAGIC = 0x31424353  # "SCB1"
VERSION = 1
HEADER_BYTES = 64
SECTIONS = ("codes_k", "codes_v", "scales_k", "scales_v", "basis_k", "basis_v", "minmax", "vnorm")
_HEADER = struct.Struct("<IHHIHHHHHHHBBi8I")
assert _HEADER.size == HEADER_BYTES


def _align16(x: int) -> int:
    return (x + 15) & ~15


def section_head_bytes(block_size, head_dim, kp_keys, kp_values, per_row):
    """Bytes of one KV head's slice of each section (minmax: K or V half)."""
    s = block_size if per_row else 1
    return [block_size * kp_keys, kp_values * block_size, 4 * s, 4 * s,
            2 * head_dim * kp_keys, 2 * head_dim * kp_values, 8, 4]


def layout(kv_heads, head_dim, block_size, kp_keys, kp_values, per_row):
    """(section offsets, record bytes) of one block record."""
    hb = section_head_bytes(block_size, head_dim, kp_keys, kp_values, per_row)
    off, offsets = HEADER_BYTES, []
    for s, b in enumerate(hb):
        off = _align16(off)
        offsets.append(off)
        off += b * kv_heads * (2 if s == 6 else 1)
    return offsets, _align16(off)


def record_bytes(kv_heads, head_dim, block_size, kp_keys, kp_values, per_row):
    return layout(kv_heads, head_dim, block_size, kp_keys, kp_values, per_row)[1]


@dataclass
class BlockHeader:
    magic: int
    version: int
    header_bytes: int
    record_bytes: int
    kv_heads: int
    head_dim: int
    block_size: int
    k_keys: int
    k_values: int
    kp_keys: int
    kp_values: int
    granularity: int
    reserved: int
    start_position: int
    offsets: List[int]

    def pack(self) -> bytes:
        return _HEADER.pack(self.magic, self.version, self.header_bytes, self.record_bytes, self.kv_heads,
                            self.head_dim, self.block_size, self.k_keys, self.k_values, self.kp_keys,
                            self.kp_values, self.granularity, self.reserved, self.start_position, *self.offsets)

    @classmethod
    def unpack(cls, buf) -> "BlockHeader":
        v = _HEADER.unpack_from(bytes(buf[:HEADER_BYTES]))
        return cls(*v[:14], list(v[14:]))

    def validate(self):
        """Raises ValueError unless this is a version-1 record whose offsets
        and size follow the layout rule for its own geometry."""
        if self.magic != MAGIC:
            raise ValueError(f"not a spectral block record (magic {self.magic:#x})")
        if self.version != VERSION or self.header_bytes != HEADER_BYTES:
            raise ValueError(f"unsupported record version {self.version} / header {self.header_bytes} bytes")
        offs, size = layout(self.kv_heads, self.head_dim, self.block_size, self.kp_keys, self.kp_values,
                            self.granularity == 1)
        if offs != self.offsets or size != self.record_bytes:
            raise ValueError("record offsets or size do not match its geometry")


def headers(buf, count=None) -> List[BlockHeader]:
    """Headers of the consecutive records in ``buf`` (bytes-like / uint8 CPU
    tensor), each validated."""
    data = bytes(buf.numpy().tobytes()) if hasattr(buf, "numpy") else bytes(buf)
    out, off = [], 0
    while off < len(data) and (count is None or len(out) < count):
        h = BlockHeader.unpack(data[off:off + HEADER_BYTES])
        h.validate()
        out.append(h)
        off += h.record_bytes
    return out
