"""The C-ABI library loads and exports every entry point include/*.h declares
(no compute calls: runs without a GPU)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?\w+\**\s+\**(sc_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_the_api():
    names = _declared_functions()
    for fn in ("sc_decode_attn", "sc_decode_workspace_size", "sc_rsvd_compress", "sc_quantize_int8",
               "sc_tier_append", "sc_tier_compress", "sc_tier_dequant", "sc_last_error", "sc_abi_version",
               "sc_block_record_bytes", "sc_tier_pack", "sc_tier_unpack", "sc_prefill_attn", "sc_block_scores",
               "sc_block_values", "sc_rope_rotate"):
        assert fn in names


def test_library_exports_every_declared_symbol():
    from unsloth_spectral import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libspectral_hip.so not built (python unsloth-spectral_amd/build.py)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for fn in _declared_functions():
        assert hasattr(lib, fn), fn
    assert set(_lib.PROTOTYPES) == _declared_functions()
    assert _lib.load().sc_abi_version() == _lib.ABI_VERSION == 6


def test_struct_layouts_match_header():
    """ctypes mirrors of the C structs: field order and 8-byte alignment."""
    from unsloth_spectral import _lib
    assert ctypes.sizeof(_lib.ScTierDesc) == 11 * 4 + 4 + 14 * 8
    assert _lib.ScTierDesc.codes_k.offset == 48
    assert _lib.ScDecodeArgs.scale.offset == 24 and _lib.ScDecodeArgs.q.offset == 32
    # query_pos_i64 sits in the tail padding after split: the size is unchanged
    assert _lib.ScDecodeArgs.query_pos_i64.offset == _lib.ScDecodeArgs.split.offset + 4
    assert ctypes.sizeof(_lib.ScDecodeArgs) == _lib.ScDecodeArgs.split.offset + 8 == 184
    assert _lib.ScCompressArgs.m.offset == 48


def test_errors_are_reported_without_a_gpu():
    from unsloth_spectral import _lib
    lib = _lib.load()
    rc = lib.sc_quantize_int8(None, 1, 1, 1, 7, None, None, None, None)
    assert rc == -1
    assert b"null" in lib.sc_last_error() or b"granularity" in lib.sc_last_error()
    args = _lib.ScDecodeArgs()
    assert lib.sc_decode_attn(ctypes.byref(args), None, 0, None) == -1
    assert b"null" in lib.sc_last_error()


def test_host_side_checks_refuse_bad_calls_without_a_gpu():
    """Argument checks that return before anything is launched."""
    from unsloth_spectral import _lib
    lib = _lib.load()
    tier = _lib.ScTierDesc()
    assert lib.sc_tier_append(ctypes.byref(tier), None, None, 0, 0, 0, None, 1, 0, None) == -1   # null tier arrays
    assert lib.sc_tier_append(None, None, None, 0, 0, 0, None, 1, 0, None) == -1
    buf = ctypes.create_string_buffer(64)
    for name in ("counters", "tail_k", "tail_v", "tail_pos"):
        setattr(tier, name, ctypes.addressof(buf))
    tier.tail_capacity, tier.head_dim = 16, 128
    assert lib.sc_tier_append(ctypes.byref(tier), None, None, 0, 0, 0, None, 1, 8, None) == -1    # unknown flag
    assert b"flags" in lib.sc_last_error()
    assert lib.sc_tier_append(ctypes.byref(tier), None, None, 0, 0, 0, None, 17, 0, None) == -5   # > ring
    assert lib.sc_block_scores(None, 0, 0, 1, 8, None, None, 2, 16, 8, 128, None, None, 128, 64, 0, None,
                               None) == -1
    assert lib.sc_block_values(None, 0, 0, 1, 8, None, None, 3, 16, 8, 128, None, None) == -1    # 8 % 3
    assert b"multiple" in lib.sc_last_error()
    assert lib.sc_block_values(None, 0, 0, 1, 8, None, None, 2, 16, 65, 128, None, None) == -2   # rank > 64
    assert lib.sc_rope_rotate(None, 0, 0, 0, None, None, 0, 0, 1, 8, 1, 120, None, None) == -2  # head_dim % 16
    assert lib.sc_rope_rotate(None, 0, 0, 0, None, None, 0, 0, 1, 8, 1, 128, None, None) == -1  # null pointers
    assert lib.sc_rope_rotate(None, 0, 0, 0, None, None, 0, 0, 1, 0, 1, 128, None, None) == 0   # nothing to do
