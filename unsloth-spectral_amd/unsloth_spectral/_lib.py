"""ctypes binding of libspectral_hip.so (the C ABI declared in include/spectral_hip.h).

The library is the only compute path of this package: if it cannot be
loaded, every entry point raises (there is no CPU or PyTorch fallback).
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libspectral_hip.so")

ABI_VERSION = 6  # SC_ABI_VERSION of include/spectral_hip.h
SC_OK = 0
SC_ROPE_ABSOLUTE, SC_ROPE_DISTANCE, SC_ROPE_NONE = 0, 1, 2
SC_QUANT_PER_HEAD, SC_QUANT_PER_ROW, SC_QUANT_PER_TENSOR = 0, 1, 2
SC_CNT_NCOLD, SC_CNT_TAIL_HEAD, SC_CNT_TAIL_LEN, SC_CNT_NEXT_POS = 0, 1, 2, 3
SC_CNT_TOTAL, SC_CNT_COMPRESSIONS, SC_CNT_STATUS = 4, 5, 6
SC_NCOUNTERS = 8
SC_APPEND_DETECT_RESET, SC_APPEND_RESET, SC_APPEND_POS_I64 = 1, 2, 4
SC_ERR_CAPACITY = -5
SC_DECODE_SCRATCH_BYTES = 32 << 20

SC_DTYPE = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}
GRANULARITY = {"per_head": SC_QUANT_PER_HEAD, "per_row": SC_QUANT_PER_ROW,
               "per_tensor": SC_QUANT_PER_TENSOR}

c_i32, c_i64, c_u64, c_f32, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p


class ScTierDesc(ctypes.Structure):
    _fields_ = [
        ("batch", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32), ("block_size", c_i32),
        ("k_keys", c_i32), ("k_values", c_i32), ("kp_keys", c_i32), ("kp_values", c_i32),
        ("max_blocks", c_i32), ("tail_capacity", c_i32), ("granularity", c_i32),
        ("codes_k", c_vp), ("codes_v", c_vp), ("scales_k", c_vp), ("scales_v", c_vp),
        ("minmax_k", c_vp), ("minmax_v", c_vp), ("vnorm", c_vp),
        ("basis_k", c_vp), ("basis_v", c_vp), ("block_start", c_vp),
        ("tail_k", c_vp), ("tail_v", c_vp), ("tail_pos", c_vp), ("counters", c_vp),
    ]


class ScDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("tier", ctypes.POINTER(ScTierDesc)),
        ("q_heads", c_i32), ("rope_mode", c_i32), ("grid_blocks", c_i32), ("grid_tail", c_i32),
        ("scale", c_f32),
        ("q", c_vp), ("q_stride_b", c_i64), ("q_stride_h", c_i64),
        ("cos", c_vp), ("sin", c_vp), ("rope_stride", c_i64), ("rope_len", c_i32), ("halves_equal", c_i32),
        ("query_pos", c_vp), ("query_pos_scalar", c_i32),
        ("mask", c_vp), ("mask_stride_b", c_i64), ("mask_stride_h", c_i64),
        ("out", c_vp), ("out_stride_b", c_i64), ("out_stride_h", c_i64),
        ("logits_out", c_vp), ("logits_stride_b", c_i64), ("logits_stride_h", c_i64),
        ("split", c_i32), ("query_pos_i64", c_i32),
    ]


class ScPrefillArgs(ctypes.Structure):
    _fields_ = [
        ("tier", ctypes.POINTER(ScTierDesc)), ("q_heads", c_i32), ("t_q", c_i32), ("scale", c_f32),
        ("q", c_vp), ("q_stride_b", c_i64), ("q_stride_h", c_i64), ("q_stride_t", c_i64),
        ("query_pos", c_vp), ("query_pos_stride_b", c_i64),
        ("cos", c_vp), ("sin", c_vp), ("rope_stride", c_i64), ("rope_len", c_i32),
        ("out", c_vp), ("out_stride_b", c_i64), ("out_stride_h", c_i64), ("out_stride_t", c_i64),
    ]


class ScCompressArgs(ctypes.Structure):
    _fields_ = [
        ("count", c_i32), ("inner", c_i32), ("rows", c_i32), ("cols", c_i32), ("rank", c_i32),
        ("oversample", c_i32), ("n_iter", c_i32), ("kp", c_i32), ("granularity", c_i32),
        ("coeff_major", c_i32), ("basis_dmajor", c_i32), ("m_dtype", c_i32),
        ("m", c_vp), ("m_stride_outer", c_i64), ("m_stride_inner", c_i64), ("m_stride_row", c_i64),
        ("omega", c_vp), ("seed", c_u64),
        ("codes", c_vp), ("codes_stride_outer", c_i64), ("codes_stride_inner", c_i64),
        ("scales", c_vp), ("scales_stride_outer", c_i64), ("scales_stride_inner", c_i64),
        ("minmax", c_vp), ("minmax_stride_outer", c_i64), ("minmax_stride_inner", c_i64),
        ("vnorm", c_vp), ("vnorm_stride_outer", c_i64), ("vnorm_stride_inner", c_i64),
        ("basis", c_vp), ("basis_stride_outer", c_i64), ("basis_stride_inner", c_i64),
        ("coeffs_out", c_vp), ("svals_out", c_vp), ("vh_out", c_vp), ("omega_out", c_vp),
        ("row_weights", c_vp), ("row_weights_stride_outer", c_i64), ("row_weights_stride_inner", c_i64),
    ]


# Exported symbols and their prototypes (mirrors include/spectral_hip.h).
PROTOTYPES = {
    "sc_decode_workspace_size": (c_i32, [ctypes.POINTER(ScDecodeArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "sc_decode_attn": (c_i32, [ctypes.POINTER(ScDecodeArgs), c_vp, ctypes.c_size_t, c_vp]),
    "sc_decode_attn_noalloc": (c_i32, [ctypes.POINTER(ScDecodeArgs), c_vp]),
    "sc_rsvd_compress": (c_i32, [ctypes.POINTER(ScCompressArgs), c_vp]),
    "sc_quantize_int8": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "sc_tier_append": (c_i32, [ctypes.POINTER(ScTierDesc), c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i32, c_i32,
                               c_vp]),
    "sc_tier_compress": (c_i32, [ctypes.POINTER(ScTierDesc), c_i32, c_i32, c_i32, c_u64, c_vp]),
    "sc_tier_dequant": (c_i32, [ctypes.POINTER(ScTierDesc), c_i32, c_i32, c_vp, c_vp, c_vp]),
    "sc_prefill_attn": (c_i32, [ctypes.POINTER(ScPrefillArgs), c_vp]),
    "sc_block_record_bytes": (ctypes.c_size_t, [ctypes.POINTER(ScTierDesc)]),
    "sc_tier_pack": (c_i32, [ctypes.POINTER(ScTierDesc), c_i32, c_i32, c_i32, c_vp, ctypes.c_size_t, c_vp]),
    "sc_tier_unpack": (c_i32, [ctypes.POINTER(ScTierDesc), c_i32, c_i32, c_i32, c_vp, ctypes.c_size_t, c_vp,
                               c_vp]),
    "sc_block_scores": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp,
                                c_i64, c_i32, c_i32, c_vp, c_vp]),
    "sc_block_values": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp,
                                c_vp]),
    "sc_rope_rotate": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp,
                               c_vp]),
    "sc_last_error": (ctypes.c_char_p, []),
    "sc_abi_version": (c_i32, []),
}

_lib = None
_lock = threading.Lock()


def load():
    """Loads the HIP library (once) and returns the ctypes handle."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python unsloth-spectral_amd/build.py` "
                    "(the spectral kernels have no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in PROTOTYPES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.sc_abi_version() != ABI_VERSION:
                raise ImportError("libspectral_hip.so ABI version mismatch")
            _lib = lib
    return _lib


class SpectralHIPError(RuntimeError):
    pass


def check(rc):
    if rc != SC_OK:
        msg = load().sc_last_error().decode(errors="replace")
        raise SpectralHIPError(f"spectral HIP call failed ({rc}): {msg}")


def require_device(t, name):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a tensor on a ROCm device (got "
                           f"{getattr(t, 'device', type(t))}); the spectral path has no CPU implementation")


def stream_of(t):
    """The current HIP stream of t's device, as a handle for the C ABI."""
    return ctypes.c_void_p(_raw_stream(t.device.index if t.device.index is not None else torch.cuda.current_device()))


# torch's raw current-stream query skips building a Stream object (a few
# microseconds per launch on the host); the public call is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or \
    (lambda index: torch.cuda.current_stream(index).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


_ws = {}


def workspace(device, nbytes):
    """A reusable per-device byte workspace (grown on demand)."""
    key = (device.type, device.index)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws[key] = buf
    return buf
