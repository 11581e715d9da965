"""Decode-attention parity: HIP kernel (through the C ABI) vs the oracle.

Bar: outputs within 2e-3 max-abs and 1e-2 of max|ref|
(FP16 out, FP32 accumulate), logits Pearson >= 0.9999 against the
FP16-faithful restatement of the same RoPE mode."""
import zlib

import numpy as np
import pytest
import torch

from gpu_helpers import cache_from_states, tables
from helpers import pearson, random_state, rope_tables
from oracle.attention import closed_form64, spectral_attention_decode as o_abs
from oracle.attention import spectral_attention_forward as o_dist

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL_MAX = 1e-2


def _run(states, Q16, cos, sin, q, mode, mask=None, block_size=None, qpos_tensor=False, split=0,
         with_logits=True):
    from unsloth_spectral import _lib
    from unsloth_spectral._decode import run_decode
    cache = cache_from_states(states, block_size)
    B, Hq, D = Q16.shape
    total = states[0].total_tokens()
    ct, st = tables(cos, sin)
    Q = torch.from_numpy(Q16).cuda().reshape(B, Hq, 1, D)
    logits = torch.full((B, Hq, total), float("nan"), dtype=torch.float32, device="cuda") if with_logits else None
    m = None if mask is None else torch.from_numpy(mask).cuda()
    qp = torch.tensor(q, dtype=torch.int32, device="cuda") if qpos_tensor else q
    code = _lib.SC_ROPE_ABSOLUTE if mode == "absolute" else _lib.SC_ROPE_DISTANCE
    out = run_decode(Q, cache, ct, st, qp, m, None, code, logits=logits, split=split)
    torch.cuda.synchronize()
    return out[:, :, 0].float().cpu().numpy(), (logits.cpu().numpy() if with_logits else None)


def _ulp16(x):
    """Spacing of fp16 numbers at |x| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _check(states, Q16, cos, sin, q, mode, mask=None, block_size=None, seqs=None, qpos_tensor=False,
           ulp_aware=False):
    """ulp_aware: for stress inputs (large, peaky scores) the reference's own
    fp16 arithmetic -- Q rotated elementwise in fp16, scores and logits cast
    to fp16 -- moves its outputs away from exact attention by more than 2e-3
    (one fp16 ulp of a score near 100 is 0.06, i.e. 5e-3 of a logit).  No
    implementation that does not replay the reference op by op can then be
    within 2e-3 of it.  The bar becomes relative to that measured noise:
    within max(2e-3, one fp16 ulp of the output, 2 x noise) of the fp16
    restatement, and no farther from the float64 closed form than
    1.5 x noise + 2e-3, where noise = max |reference - closed form|."""
    out, logits = _run(states, Q16, cos, sin, q, mode, mask, block_size, qpos_tensor)
    fn = o_abs if mode == "absolute" else o_dist
    qs = q if isinstance(q, (list, tuple)) else [q] * len(states)
    for b in (seqs if seqs is not None else range(len(states))):
        mb = None if mask is None else mask[b]
        ref, _, logits16 = fn(Q16[b], states[b], cos, sin, qs[b], mask=mb)
        ref = ref.astype(np.float64)
        err = np.abs(out[b] - ref).max()
        if ulp_aware:
            exact, _ = closed_form64(Q16[b], states[b], cos, sin, qs[b], mask=mb, mode=mode)
            noise = np.abs(ref - exact).max()
            tol = np.maximum(np.maximum(ATOL, _ulp16(ref)), 2.0 * noise)
            assert np.all(np.abs(out[b] - ref) <= tol), (b, err, noise)
            assert np.abs(out[b] - exact).max() <= 1.5 * noise + ATOL, (b, np.abs(out[b] - exact).max(), noise)
        else:
            assert err <= ATOL, (b, err)
        assert err <= RTOL_MAX * np.abs(ref).max(), (b, err, np.abs(ref).max())
        lg = logits[b]
        keep = np.isfinite(logits16.astype(np.float64)) if mb is None else (np.broadcast_to(mb, lg.shape) != 0)
        assert np.isfinite(lg[keep]).all()
        assert pearson(lg[keep], logits16[keep]) >= 0.9999, b
    return out, logits


CASES = [
    # H_kv, rep, D, nblk, T, kK, kV, tail
    (2, 4, 128, 2, 128, 16, 32, 100),
    (2, 4, 128, 3, 256, 32, 32, 64),
    (4, 1, 64, 2, 128, 16, 16, 63),
    (2, 2, 128, 1, 512, 64, 64, 1),
    (1, 8, 64, 2, 64, 32, 16, 0),
    (2, 4, 128, 0, 512, 16, 32, 511),
    (2, 16, 128, 1, 128, 32, 32, 512),
]


@pytest.mark.parametrize("mode", ["absolute", "distance"])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("case", CASES)
def test_decode_small_cases(mode, per_row, case):
    H, rep, D, nblk, T, kK, kV, tail = case
    rng = np.random.default_rng(zlib.crc32(repr((mode, per_row) + case).encode()))
    B = 2
    states = [random_state(rng, H, D, nblk, T, kK, kV, tail, per_row=per_row) for _ in range(B)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 16, D)
    Q = rng.standard_normal((B, H * rep, D)).astype(np.float16)
    print(f"case={case} mode={mode} per_row={per_row}", flush=True)
    _check(states, Q, cos, sin, total - 1, mode, block_size=T)


def test_golden_tiny_fixture():
    import os
    from golden_io import load_decode_case
    case = load_decode_case(os.path.join(os.path.dirname(__file__), "golden", "decode_tiny.npz"))
    for mode in ("absolute", "distance"):
        out, _ = _run([case["state"]], case["Q"][None], case["cos"], case["sin"], case["q"], mode, block_size=128)
        assert np.abs(out[0] - case[f"out64_{mode}"]).max() < ATOL


@pytest.mark.parametrize("mode", ["absolute", "distance"])
def test_mask_and_peaky_scores(mode):
    rng = np.random.default_rng(7)
    H, rep, D = 2, 4, 128
    states = [random_state(rng, H, D, 2, 256, 16, 32, 80, coeff_std=3.0, tail_std=1.5) for _ in range(2)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 16, D)
    Q = (rng.standard_normal((2, H * rep, D)) * 2.5).astype(np.float16)
    mask = (rng.random((2, H * rep, total)) > 0.25).astype(np.uint8)
    _check(states, Q, cos, sin, total - 1, mode, mask=mask, block_size=256, ulp_aware=True)


def test_per_sequence_query_positions_on_device():
    rng = np.random.default_rng(8)
    states = [random_state(rng, 2, 128, 2, 128, 16, 32, 50, start=s) for s in (0, 1000)]
    cos, sin = rope_tables(2000, 128)
    Q = rng.standard_normal((2, 8, 128)).astype(np.float16)
    q = [states[0].total_tokens() - 1, 1000 + states[1].total_tokens() - 1]
    _check(states, Q, cos, sin, q, "distance", block_size=128, qpos_tensor=True)


def test_int64_query_positions_equal_int32():
    """A model's int64 position ids reach the kernel as they are
    (query_pos_i64, no conversion launch): the same output bits as int32
    positions, which the oracle check above covers; a strided int64 view is
    converted instead and gives the same bits too."""
    from unsloth_spectral import _lib
    from unsloth_spectral._decode import run_decode
    rng = np.random.default_rng(18)
    states = [random_state(rng, 2, 128, 2, 128, 16, 32, 50, start=s) for s in (0, 1000)]
    cos, sin = rope_tables(2000, 128)
    Q16 = rng.standard_normal((2, 8, 128)).astype(np.float16)
    q = [states[0].total_tokens() - 1, 1000 + states[1].total_tokens() - 1]
    _check(states, Q16, cos, sin, q, "distance", block_size=128, qpos_tensor=True)
    cache = cache_from_states(states, 128)
    ct, st = tables(cos, sin)
    Q = torch.from_numpy(Q16).cuda().reshape(2, 8, 1, 128)
    code = _lib.SC_ROPE_DISTANCE
    ref = run_decode(Q, cache, ct, st, torch.tensor(q, dtype=torch.int32, device="cuda"), None, None, code)
    ids = torch.tensor([[p] for p in q], dtype=torch.int64, device="cuda")        # [B, 1] like a model's
    got = run_decode(Q, cache, ct, st, ids[:, -1], None, None, code)
    wide = torch.tensor([[0, p] for p in q], dtype=torch.int64, device="cuda")    # [:, -1] has stride 2
    got2 = run_decode(Q, cache, ct, st, wide[:, -1], None, None, code)
    torch.cuda.synchronize()
    assert torch.equal(got, ref) and torch.equal(got2, ref)


def test_unequal_table_halves_use_full_rows():
    rng = np.random.default_rng(9)
    states = [random_state(rng, 2, 128, 2, 128, 16, 32, 40)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 4, 128)
    cos = cos.copy()
    sin = sin.copy()
    cos[:, 64:] = (cos[:, 64:].astype(np.float32) * 0.9).astype(np.float16)   # e.g. scaled RoPE variants
    sin[:, 64:] = (sin[:, 64:].astype(np.float32) * 1.1).astype(np.float16)
    Q = rng.standard_normal((1, 8, 128)).astype(np.float16)
    _check(states, Q, cos, sin, total - 1, "absolute", block_size=128)
    _check(states, Q, cos, sin, total - 1, "distance", block_size=128)


def test_c1_geometry():
    """Mistral-7B heads, batch 1, ctx 4096: 7 cold blocks (k=16) + 512 tail."""
    rng = np.random.default_rng(10)
    states = [random_state(rng, 8, 128, 7, 512, 16, 16, 512)]
    cos, sin = rope_tables(4096 + 64, 128)
    Q = rng.standard_normal((1, 32, 128)).astype(np.float16)
    for mode in ("absolute", "distance"):
        _check(states, Q, cos, sin, 4095, mode)


def test_c3_geometry_full_batch():
    """Batch 8, ctx 16384: 31 cold blocks (k=32, per-row scales) + 512 tail.
    Two sequences against the oracle; the others via batch invariance."""
    rng = np.random.default_rng(11)
    states = [random_state(rng, 8, 128, 31, 512, 32, 32, 512, per_row=True) for _ in range(8)]
    cos, sin = rope_tables(16384 + 64, 128)
    Q = rng.standard_normal((8, 32, 128)).astype(np.float16)
    out, logits = _check(states, Q, cos, sin, 16383, "absolute", seqs=[0, 7])
    # batch invariance at a fixed split: sequence 3 alone == sequence 3 in
    # the batch (batch 8 fills the GPU unsplit; batch 1 alone would split)
    out1, logits1 = _run([states[3]], Q[3:4], cos, sin, 16383, "absolute", split=1)
    np.testing.assert_array_equal(out1[0], out[3])
    np.testing.assert_array_equal(logits1[0], logits[3])


@pytest.mark.parametrize("with_logits", [False, True])
def test_block_split_variants(with_logits):
    """A cold block split over 1, 2, 4 or 8 workgroups (64-token ranges
    each) gives the oracle's result; splits differ from each other only in
    where partial sums are rounded (each workgroup's record is merged in
    fp32 and the output rounded once to fp16): within a few fp16 ulps of
    the largest output.  Without
    logits this is the branch-free path, with logits the general one."""
    from unsloth_spectral._lib import SpectralHIPError
    rng = np.random.default_rng(14)
    states = [random_state(rng, 8, 128, 3, 512, 32, 32, 200, per_row=True) for _ in range(2)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 16, 128)
    Q = rng.standard_normal((2, 32, 128)).astype(np.float16)
    outs = {}
    for split in (1, 2, 4, 8, 0):
        out, lg = _run(states, Q, cos, sin, total - 1, "absolute", split=split, with_logits=with_logits)
        outs[split] = out
        for b in range(2):
            ref, _, logits16 = o_abs(Q[b], states[b], cos, sin, total - 1)
            assert np.abs(out[b] - ref).max() <= ATOL, (split, b)
            if with_logits:
                assert pearson(lg[b].ravel(), logits16.ravel()) >= 0.9999
        diff = np.abs(out - outs[1]).max()
        assert diff <= 4 * _ulp16(np.abs(outs[1]).max()), (split, diff)
    assert np.array_equal(outs[0], outs[8])   # 2 sequences x 2 head groups x 3 blocks: auto splits 8 ways
    with pytest.raises(SpectralHIPError):
        _run(states, Q, cos, sin, total - 1, "absolute", split=3, with_logits=with_logits)


@pytest.mark.parametrize("nblk", [9, 33])
def test_records_merged_over_several_chunks(nblk):
    """72 or 264 partial records per query head (9 or 33 cold blocks split
    over 8 workgroups each): the combine's waves take 64 records per round
    (2 waves for 72 records, the second chunk partly filled; 4 waves for 264,
    wave 0 taking two rounds) and wave 0 merges their states.  Outputs meet
    the oracle's bar; split 1 (one record per block + tail tiles) agrees
    within a few fp16 ulps."""
    rng = np.random.default_rng(21 + nblk)
    states = [random_state(rng, 2, 128, nblk, 512, 16, 32, 100)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 8, 128)
    Q = rng.standard_normal((1, 8, 128)).astype(np.float16)
    ref, _, _ = o_abs(Q[0], states[0], cos, sin, total - 1)
    out8, _ = _run(states, Q, cos, sin, total - 1, "absolute", split=8, with_logits=False)
    out1, _ = _run(states, Q, cos, sin, total - 1, "absolute", split=1, with_logits=False)
    ref = ref.astype(np.float64)
    assert np.abs(out8[0] - ref).max() <= ATOL
    assert np.abs(out8[0] - ref).max() <= RTOL_MAX * np.abs(ref).max()
    assert np.abs(out8[0] - out1[0]).max() <= 4 * _ulp16(np.abs(out1[0]).max())


def test_rope_none_equals_dense_unrotated():
    from unsloth_spectral import _lib
    from unsloth_spectral._decode import run_decode
    rng = np.random.default_rng(12)
    states = [random_state(rng, 2, 128, 2, 128, 16, 32, 30)]
    cache = cache_from_states(states, 128)
    Q = rng.standard_normal((1, 8, 128)).astype(np.float16)
    out = run_decode(torch.from_numpy(Q).cuda()[:, :, None], cache, None, None, 0, None, None, _lib.SC_ROPE_NONE)
    K, V = states[0].get_kv()
    Kr = np.repeat(K.astype(np.float64), 4, 0)
    Vr = np.repeat(V.astype(np.float64), 4, 0)
    lg = np.einsum("hd,htd->ht", Q[0].astype(np.float64), Kr) / np.sqrt(128)
    p = np.exp(lg - lg.max(-1, keepdims=True))
    ref = np.einsum("ht,htd->hd", p / p.sum(-1, keepdims=True), Vr)
    assert np.abs(out[0, :, 0].float().cpu().numpy() - ref).max() < ATOL


def test_public_entry_points_and_reference_style_cache():
    """spectral_attention_decode / forward accept a reference-style cache
    object (SpectralBlock list with fp16 coefficients and [min, max])."""
    import types
    from unsloth_spectral import SpectralBlock, spectral_attention_decode, spectral_attention_forward
    rng = np.random.default_rng(13)
    st = random_state(rng, 2, 128, 2, 128, 16, 32, 20)
    blocks = []
    for b in st.blocks:
        ck, cv = b.coeffs_k(), b.coeffs_v()
        mm = lambda c: torch.from_numpy(np.stack([c.astype(np.float32).min(axis=(1, 2)),   # noqa: E731
                                                  c.astype(np.float32).max(axis=(1, 2))], -1)).cuda()
        blocks.append(SpectralBlock(torch.from_numpy(ck).cuda(), torch.from_numpy(b.basis_k).cuda(),
                                    torch.from_numpy(cv).cuda(), torch.from_numpy(b.basis_v).cuda(),
                                    mm(ck), mm(cv), b.T, b.start))
    hk = torch.from_numpy(st.tail_k).cuda()[None]
    hv = torch.from_numpy(st.tail_v).cuda()[None]
    ref_cache = types.SimpleNamespace(num_heads=2, hot_position_ids=torch.from_numpy(st.tail_pos).cuda()[None],
                                      get_spectral_components=lambda: (blocks, hk, hv))
    total = st.total_tokens()
    cos, sin = rope_tables(total + 4, 128)
    ct, stt = tables(cos, sin)
    Q = rng.standard_normal((1, 8, 1, 128)).astype(np.float16)
    Qt = torch.from_numpy(Q).cuda()
    for fn, ofn in ((spectral_attention_decode, o_abs), (spectral_attention_forward, o_dist)):
        out = fn(Qt, ref_cache, ct, stt, total - 1)
        ref, _, _ = ofn(Q[0, :, 0], st, cos, sin, total - 1)
        assert out.shape == (1, 8, 1, 128) and out.dtype == torch.float16
        assert np.abs(out[0, :, 0].float().cpu().numpy() - ref.astype(np.float64)).max() < ATOL


def test_empty_cache_raises():
    from unsloth_spectral import SpectralCache, spectral_attention_decode
    c = SpectralCache(2, 128, batch_size=1)
    cos, sin = tables(*rope_tables(16, 128))
    with pytest.raises(ValueError):
        spectral_attention_decode(torch.zeros(1, 8, 1, 128, dtype=torch.float16, device="cuda"), c, cos, sin, 0)


# ---------------------------------------------------------------- branch-free path
# sc_decode_attn runs its branch-free instantiation (the one the benchmark
# times) when no mask and no logits are requested, RoPE is absolute or
# distance over a table with equal halves, the KV heads are a multiple of 4
# and the GQA group holds at most 4 query heads.  These tests ask for no
# logits, so that path is the one compared with the oracle; the logits of
# the Pearson check come from a second call with logits (the general path)
# on the same tiers, whose output is checked as well.

def _check_fast(states, Q16, cos, sin, q, mode, block_size=None, seqs=None, split=0):
    out, _ = _run(states, Q16, cos, sin, q, mode, block_size=block_size, split=split, with_logits=False)
    out_g, logits = _run(states, Q16, cos, sin, q, mode, block_size=block_size, split=split, with_logits=True)
    fn = o_abs if mode == "absolute" else o_dist
    for b in (seqs if seqs is not None else range(len(states))):
        ref, _, logits16 = fn(Q16[b], states[b], cos, sin, q)
        ref = ref.astype(np.float64)
        for o in (out[b], out_g[b]):
            err = np.abs(o - ref).max()
            assert err <= ATOL, (b, err)
            assert err <= RTOL_MAX * np.abs(ref).max(), (b, err, np.abs(ref).max())
        assert np.isfinite(logits[b]).all()
        assert pearson(logits[b], logits16) >= 0.9999, b
    return out, out_g, logits


@pytest.mark.parametrize("mode", ["absolute", "distance"])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("ranks", [(16, 16), (16, 32), (32, 32)])
def test_fast_path_modes_scales_ranks(mode, per_row, ranks):
    """8 KV heads / 32 query heads, 3 blocks of 512 + a 200-token tail, two
    sequences with different data."""
    kK, kV = ranks
    rng = np.random.default_rng(zlib.crc32(repr(("fast", mode, per_row, ranks)).encode()))
    states = [random_state(rng, 8, 128, 3, 512, kK, kV, 200, per_row=per_row, batched_qr=True) for _ in range(2)]
    total = states[0].total_tokens()
    cos, sin = rope_tables(total + 16, 128)
    Q = rng.standard_normal((2, 32, 128)).astype(np.float16)
    print(f"fast path mode={mode} per_row={per_row} ranks={ranks}", flush=True)
    _check_fast(states, Q, cos, sin, total - 1, mode)


@pytest.mark.parametrize("per_row", [False, True])
def test_fast_path_c1_geometry(per_row):
    """Batch 1, 4096 context: 7 cold blocks k=16 + 512 tail, both modes."""
    rng = np.random.default_rng(40 + per_row)
    states = [random_state(rng, 8, 128, 7, 512, 16, 16, 512, per_row=per_row, batched_qr=True)]
    cos, sin = rope_tables(4096 + 64, 128)
    Q = rng.standard_normal((1, 32, 128)).astype(np.float16)
    for mode in ("absolute", "distance"):
        print(f"C1 fast path per_row={per_row} mode={mode}", flush=True)
        _check_fast(states, Q, cos, sin, 4095, mode)


@pytest.mark.parametrize("mode", ["absolute", "distance"])
def test_fast_path_c3_geometry(mode):
    """Batch 8, 16384 context: 31 cold blocks k=32 per row + 512 tail.  Two
    sequences against the oracle; every other one equals itself decoded
    alone at the same split (batch invariance)."""
    rng = np.random.default_rng(50 + (mode == "distance"))
    states = [random_state(rng, 8, 128, 31, 512, 32, 32, 512, per_row=True, batched_qr=True) for _ in range(8)]
    cos, sin = rope_tables(16384 + 64, 128)
    Q = rng.standard_normal((8, 32, 128)).astype(np.float16)
    print(f"C3 fast path mode={mode}", flush=True)
    out, _, _ = _check_fast(states, Q, cos, sin, 16383, mode, seqs=[0, 5], split=1)
    for b in (1, 2, 3, 4, 6, 7):
        alone, _ = _run([states[b]], Q[b:b + 1], cos, sin, 16383, mode, split=1, with_logits=False)
        np.testing.assert_array_equal(alone[0], out[b])


def test_fast_path_c5_geometry():
    """Batch 16, 64 cold blocks k=32 (per row) + 512 tail = 33,280 context,
    absolute RoPE.  Four distinct sequences (each used four times); two
    compared with the oracle, the rest by batch invariance."""
    rng = np.random.default_rng(60)
    distinct = [random_state(rng, 8, 128, 64, 512, 32, 32, 512, per_row=True, batched_qr=True) for _ in range(4)]
    states = [distinct[b % 4] for b in range(16)]
    ctx = 64 * 512 + 512
    cos, sin = rope_tables(ctx + 64, 128)
    Q = rng.standard_normal((16, 32, 128)).astype(np.float16)
    print("C5 fast path", flush=True)
    out, _, _ = _check_fast(states, Q, cos, sin, ctx - 1, "absolute", seqs=[0, 9])
    for b in (3, 14):
        alone, _ = _run([states[b]], Q[b:b + 1], cos, sin, ctx - 1, "absolute", split=1, with_logits=False)
        np.testing.assert_array_equal(alone[0], out[b])
