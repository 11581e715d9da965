"""Query rotation (sc_rope_rotate) against the fp16 tensor expression of the
reference's apply_rotary_pos_emb (integration.py:428-465): bit-identical.

Queries are strided views of a projection output ([B, T, H, D] transposed to
[B, H, T, D]), as the patched attention passes them; cos/sin are per-sequence
rows [B, T, D] (the model's position embeddings) or one set [T, D] shared by
the batch."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _expr(q, cos, sin):
    from unsloth_spectral.integration import rotate_half
    if cos.dim() == 2:
        cos, sin = cos[None], sin[None]
    return q * cos[:, None] + rotate_half(q) * sin[:, None]


def _tables(B, T, D, theta, g, shared):
    pos = torch.randint(0, 40000, (1 if shared else B, T), generator=g).cuda()
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, device="cuda").float() / D))
    emb = torch.cat([pos[..., None].float() * inv] * 2, dim=-1)
    cos, sin = emb.cos().half(), emb.sin().half()
    return (cos[0], sin[0]) if shared else (cos, sin)


@pytest.mark.parametrize("B,H,T,D,shared", [(1, 32, 1, 128, False), (2, 8, 3, 128, False), (3, 4, 5, 64, True),
                                            (2, 2, 7, 256, False), (4, 8, 1, 16, True)])
def test_rotation_is_bit_identical_to_the_tensor_expression(B, H, T, D, shared):
    from unsloth_spectral.integration import _rotate_queries
    g = torch.Generator().manual_seed(B * 1000 + H * 10 + T)
    x = (torch.randn(B, T, H, D, generator=g) * 30).half().cuda()   # large values: rounding matters
    q = x.transpose(1, 2)                                           # strided [B, H, T, D]
    cos, sin = _tables(B, T, D, 1e6, g, shared)
    got = _rotate_queries(q, cos, sin)
    want = _expr(q, cos, sin)
    assert got.is_contiguous() and got.dtype == torch.float16
    assert torch.equal(got, want), (got.float() - want.float()).abs().max().item()


def test_c_abi_call_and_argument_checks():
    from unsloth_spectral import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(3)
    B, H, T, D = 2, 4, 2, 128
    q = torch.randn(B, H, T, D, generator=g).half().cuda()
    cos, sin = _tables(B, T, D, 1e4, g, False)
    out = torch.full_like(q, float("nan"))
    stream = _lib.stream_of(q)
    assert lib.sc_rope_rotate(_lib.ptr(q), q.stride(0), q.stride(1), q.stride(2), _lib.ptr(cos), _lib.ptr(sin),
                              cos.stride(0), cos.stride(1), B, H, T, D, _lib.ptr(out), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, _expr(q, cos, sin))
    # a misaligned row stride is refused before anything is launched
    assert lib.sc_rope_rotate(_lib.ptr(q), q.stride(0), q.stride(1), 4, _lib.ptr(cos), _lib.ptr(sin),
                              cos.stride(0), cos.stride(1), B, H, T, D, _lib.ptr(out), stream) == -1
    assert b"aligned" in lib.sc_last_error()
