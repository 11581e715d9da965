"""Benchmark: spectral decode attention + rSVD block compression on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--rotate R] [--only-headline]
    python bench.py --model-loop [--prompt 8192] [--decode-steps 256]
    python bench.py ... --copy-probe-mib 256          (under rocprofv3 --pmc: calibration kernel)
    python bench.py --summarize-pmc FETCH_DIR WRITE_DIR --copy-probe-mib 256

Workloads (synthetic data, seeds fixed; 32 query / 8 KV heads, head_dim 128,
absolute RoPE theta 1e6, one FP32 INT8 scale per row, 512-token blocks):
  decode (headline)  batch 8, context 16384 = 31 cold blocks (INT8 codes k=32,
          FP16 bases) + 512 FP16 tail tokens per sequence.  K/V are
          U diag(exp(-i/8)) V^T + N(0, 0.01^2) per (sequence, KV head); the
          cold blocks are compressed on the GPU by this library's rSVD (k=32,
          p=5, q=2) before timing.  One step = one decode-attention call for
          one layer.  R distinct tier sets (default 4, ~490 MB of tiers) are
          rotated so that the 256 MB MALL cannot hold the working set.
  decode, batch 1    context 4096 = 7 cold blocks k=16 + 512 tail (latency bound).
  decode, batch 16   context 33280 = 64 cold blocks k=32 + 512 tail; also the
          stall of one block compression (a token that fills the tail:
          append + compress + decode, minus a step that does not compress).
  rsvd    8 x 512 x 128 FP16 blocks of the same distribution, k=16, p=5, q=2,
          per-row INT8 quantisation; blocks/sec = matrices per second.
  prefill  one layer of an 8192-token prompt (batch 1) attending causally over
          its 16 cold blocks (k=16): the HIP prefill kernel against the dense
          reference path (get_kv + fp16 attention).
  model loop (--model-loop, separate JSON line)  transformers
          MistralForCausalLM with Mistral-7B's shape (32 layers, hidden 4096,
          32/8 heads, FFN 14336, vocab 32768), random FP16 weights, patched
          with patch_unsloth_attention (k=16): 8192-token prompt, then 256
          greedy decode steps; the same model with transformers' dense FP16
          KV cache runs beside it.
Prints one JSON line.  value = algorithmic HBM bytes of one headline decode
call divided by the measured time per step (GB/s); roofline.achieved uses the
event-timed duration of the decode call itself (partial + combine kernels).
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "unsloth-spectral_amd"))
os.environ.setdefault("UNSLOTH_SPECTRAL_QUIET", "1")

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA

B, HQ, HKV, D, TB, NBLK, K_RANK, TAIL = 8, 32, 8, 128, 512, 31, 32, 512
CTX = NBLK * TB + TAIL


def log(msg):
    """Progress line on stderr (stdout carries only the JSON result)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bytes(B, H, nblk, k_k, k_v, tail, per_row=True, hq=32, d=128, tb=512):
    """Algorithmic bytes of one decode call: INT8 codes + scales + FP16 bases
    + FP16 tail K,V + FP16 Q in / O out."""
    scales = tb * 4 * 2 if per_row else 2 * 4
    per_bh = nblk * tb * (k_k + k_v) + nblk * scales + nblk * (k_k + k_v) * d * 2 + tail * d * 2 * 2
    return B * H * per_bh + 2 * B * hq * d * 2


class Hip:
    """Minimal HIP runtime access for events on the launch stream."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.lib.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        self.lib.hipEventSynchronize(b)
        ms = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


def lowrank_kv(torch, seed, n, ctx, d, device, unit_scale=False):
    """n matrices U diag(sigma) V^T + 0.01 N(0,1), sigma_i = exp(-i/8), U and V
    the Q factors of Gaussian draws.  Generated on the host (seeded CPU
    generator, LAPACK QR) so the data do not depend on the GPU's libraries."""
    g = torch.Generator()
    g.manual_seed(seed)
    sig = torch.exp(-torch.arange(d, dtype=torch.float32) / 8.0)
    lift = math.sqrt(ctx * d / float((sig ** 2).sum())) if unit_scale else 1.0
    out = torch.empty(n, ctx, d, dtype=torch.float16, device=device)
    for i in range(n):
        U, _ = torch.linalg.qr(torch.randn(ctx, d, generator=g))
        V, _ = torch.linalg.qr(torch.randn(d, d, generator=g))
        out[i] = ((U * (sig * lift)) @ V.T + 0.01 * torch.randn(ctx, d, generator=g)).half().to(device)
    return out


def orthonormal_columns(torch, X, passes=2):
    """Orthonormal basis of the column space of each X [m, n, k] (n >= k):
    CholeskyQR, twice.  The Gram matrices X^T X are formed in float64 on the
    device; their k x k Cholesky factors and inverses are computed on the
    host (LAPACK).  With positive Cholesky diagonals this is the Q factor of
    QR with a positive R diagonal, so the distribution equals lowrank_kv's
    (a Haar-distributed basis).  The device's own QR solver is not used."""
    X = X.to(torch.float64)
    for _ in range(passes):
        G = torch.matmul(X.transpose(1, 2).contiguous(), X)
        L = torch.linalg.cholesky(G.cpu())
        Rinv = torch.linalg.inv(L.transpose(1, 2))
        X = torch.matmul(X, Rinv.to(X.device))
    return X


def lowrank_kv_device(torch, seed, n, ctx, d, device, chunk=16):
    """Same distribution as lowrank_kv, drawn on the GPU (seeded device
    generator, orthonormalised by orthonormal_columns) for the large batch-16
    workload."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    sig = torch.exp(-torch.arange(d, dtype=torch.float64, device=device) / 8.0)
    out = torch.empty(n, ctx, d, dtype=torch.float16, device=device)
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        U = orthonormal_columns(torch, torch.randn(m, ctx, d, generator=g, device=device))
        V = orthonormal_columns(torch, torch.randn(m, d, d, generator=g, device=device))
        out[i:i + m] = (torch.matmul(U * sig, V.transpose(1, 2).contiguous())
                        + 0.01 * torch.randn(m, ctx, d, generator=g, device=device, dtype=torch.float64)).half()
        del U, V
    return out


def build_decode(torch, device, b, nblk, k, tail, on_device=False, max_blocks=None):
    """Tier state of a decode workload (b sequences, nblk cold blocks of rank
    k, tail FP16 tokens), the cold blocks compressed by the HIP rSVD."""
    from unsloth_spectral import SpectralCache, compress_matrices
    ctx = nblk * TB + tail
    gen = lowrank_kv_device if on_device else lowrank_kv
    Kx = gen(torch, 2, b * HKV, ctx, D, device)
    Vx = gen(torch, 3, b * HKV, ctx, D, device)
    cold = nblk * TB
    tiers = []
    for X, seed in ((Kx, 4), (Vx, 5)):
        M = X[:, :cold].reshape(b * HKV * nblk, TB, D)
        r = compress_matrices(M, k, seed=seed, granularity="per_row")
        tiers.append((r["codes"].view(b, HKV, nblk, TB, -1)[..., :k],
                      r["scales"].view(b, HKV, nblk, TB),
                      r["basis"].view(b, HKV, nblk, -1, D)[:, :, :, :k],
                      r["minmax"].view(b, HKV, nblk, 2)))
    (ck, sk, bk, mk), (cv, sv, bv, mv) = tiers
    start = (torch.arange(nblk, device=device) * TB)[None].expand(b, nblk)
    tk = Kx[:, cold:].reshape(b, HKV, tail, D)
    tv = Vx[:, cold:].reshape(b, HKV, tail, D)
    tp = torch.arange(cold, ctx, device=device)[None].expand(b, tail)
    cache = SpectralCache.from_tiers(ck, sk, bk, cv, sv, bv, start, tk, tv, tp, block_size=TB,
                                     tail_capacity=2 * TB, minmax_k=mk, minmax_v=mv, max_blocks=max_blocks)
    return cache, (Kx, Vx), tiers


def build_c3(torch, device):
    cache, raw, _ = build_decode(torch, device, B, NBLK, K_RANK, TAIL)
    return cache, raw


def rope_tables(torch, length, device, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=device, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(length, device=device, dtype=torch.float32), inv)
    emb = torch.cat([emb, emb], dim=-1)
    return emb.cos().half().contiguous(), emb.sin().half().contiguous()


def decode_args(lib_mod, cache, Q, out, cos, sin, qpos, split=0):
    a = lib_mod.ScDecodeArgs()
    a.split = split
    tier = cache._tier()
    a.tier = ctypes.pointer(tier)
    a.q_heads, a.rope_mode = HQ, lib_mod.SC_ROPE_ABSOLUTE
    a.grid_blocks, a.grid_tail = cache.num_cold_blocks, cache.hot_len
    a.scale = 1.0 / math.sqrt(D)
    a.q, a.q_stride_b, a.q_stride_h = Q.data_ptr(), Q.stride(0), Q.stride(1)
    a.cos, a.sin, a.rope_stride, a.rope_len, a.halves_equal = cos.data_ptr(), sin.data_ptr(), D, cos.shape[0], 1
    a.query_pos_scalar = qpos
    a.out, a.out_stride_b, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    return a, tier


def cpu_decode_baseline(cache, Q, cos, sin, mode="absolute", seqs=None):
    """The oracle (fp16-faithful restatement of spectral_attention_decode,
    absolute RoPE, or of spectral_attention_forward, distance RoPE) on the
    same workload, timed on the host cores: each sequence as an independent
    batch-1 cache (the reference's cache holds one sequence), one call each.
    ``seqs`` bounds the sample to the first sequences of the batch (the rate
    is per the sample's own bytes)."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    sys.path.insert(0, HERE)
    from oracle.attention import ColdBlock, TierState, spectral_attention_decode, spectral_attention_forward
    fn = spectral_attention_decode if mode == "absolute" else spectral_attention_forward
    cores = len(os.sched_getaffinity(0))
    nb, kK, kV = cache.num_cold_blocks, cache.k_rank_keys, cache.k_rank_values
    B = Q.shape[0] if seqs is None else min(seqs, Q.shape[0])
    ctx = nb * TB + cache.hot_len
    c, s = cos.cpu().numpy(), sin.cpu().numpy()
    hot_pos = cache.hot_position_ids.cpu().numpy()
    states = []
    for b in range(B):
        ck = cache.codes_k[b, :, :nb, :, :kK].cpu().numpy()
        cv = cache.codes_v[b, :, :nb, :kV, :].transpose(-1, -2).cpu().numpy()
        sk = cache.scales_k[b, :, :nb].cpu().numpy()
        sv = cache.scales_v[b, :, :nb].cpu().numpy()
        bk = cache.basis_k[b, :, :nb, :, :kK].transpose(-1, -2).cpu().numpy()
        bv = cache.basis_v[b, :, :nb, :, :kV].transpose(-1, -2).cpu().numpy()
        blocks = [ColdBlock(ck[:, j], sk[:, j], bk[:, j], cv[:, j], sv[:, j], bv[:, j], j * TB) for j in range(nb)]
        states.append(TierState(blocks, cache.hot_K[b].cpu().numpy(), cache.hot_V[b].cpu().numpy(), hot_pos[b]))
    q = Q.reshape(Q.shape[0], HQ, D).cpu().numpy()
    with threadpool_limits(cores):
        blas = [i.get("num_threads") for i in threadpool_info()]
        t0 = time.perf_counter()
        for b in range(B):
            fn(q[b], states[b], c, s, ctx - 1)
        sec = time.perf_counter() - t0
    nbytes = decode_bytes(B, HKV, nb, kK, kV, cache.hot_len, per_row=cache.quant_granularity == "per_row")
    whole = "all" if B == Q.shape[0] else f"{B} of the {Q.shape[0]}"
    return {"value": round(nbytes / sec / 1e9, 4), "unit": "GB/s", "cores": max(b for b in blas if b) if blas else 1,
            "kind": "port", "rope": mode, "us_per_sequence": round(sec / B * 1e6, 1),
            "sample": f"oracle {fn.__name__} (fp16-faithful numpy restatement), {whole} sequences of one layer "
                      f"(context {ctx}, {nb} cold blocks k={kK}/{kV}) as independent batch-1 caches, one call "
                      f"each ({sec:.2f} s in all)"}


def rsvd_rank32_parity(torch, M):
    """Reconstruction error of the HIP rSVD at k=32 (r=37, the rank the
    16K/33K workloads compress with) against the oracle's two restatements
    with the same sketch: randomized_svd_ref (float32, no
    re-orthonormalisation between power iterations, as rsvd.py:100-113) and
    randomized_svd_subspace64 (the same subspace in float64).  Relative
    differences (e_gpu - e_oracle) / e_oracle, per matrix."""
    import numpy as np
    sys.path.insert(0, HERE)
    from oracle.rsvd import per_matrix_error, randomized_svd_ref, randomized_svd_subspace64
    from unsloth_spectral import compress_matrices
    g = torch.Generator().manual_seed(9)
    omega = torch.randn(M.shape[0], D, 37, generator=g)
    res = compress_matrices(M, 32, omega=omega.to(M.device), granularity="per_row", debug=True)
    Mn = M.cpu().numpy()
    e_gpu = per_matrix_error(Mn, res["coeffs"].cpu().numpy(), res["vh"].cpu().numpy())
    out = {}
    for name, fn in (("randomized_svd_ref", randomized_svd_ref), ("randomized_svd_subspace64", randomized_svd_subspace64)):
        U, S, Vh = fn(Mn, 32, omega.numpy())
        e = per_matrix_error(Mn, U * S[:, None, :], Vh)
        rel = (e_gpu - e) / e
        sig = lambda x: float(f"{float(x):.3e}")   # noqa: E731  (relative differences are ~1e-7)
        out[name] = {"recon_err": round(float(e.mean()), 7), "rel_diff_mean": sig(rel.mean()),
                     "rel_diff_min": sig(rel.min()), "rel_diff_max": sig(rel.max())}
    out["gpu_recon_err"] = round(float(e_gpu.mean()), 7)
    out["note"] = ("8 blocks 512x128 of the benchmark distribution, one fixed sketch; a negative difference "
                   "means the HIP fit is closer than the oracle's")
    return out


def bench_rsvd(torch, hip, device, reps=20):
    from unsloth_spectral import compress_matrices
    M = lowrank_kv(torch, 6, 8, TB, D, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        compress_matrices(M, 16, seed=7, granularity="per_row")
    torch.cuda.synchronize()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for i in range(reps):
        compress_matrices(M, 16, seed=7 + i, granularity="per_row")
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1) / reps
    r = 21
    gemm_flops = 2 * TB * D * r * (1 + 2 * 2) + 2 * r * TB * D  # M Om, 2 x (M^T Y, M Z), Q^T M
    # reconstruction error with a fixed Gaussian sketch (the oracle uses the same one)
    g = torch.Generator().manual_seed(8)
    omega = torch.randn(8, D, r, generator=g)
    res = compress_matrices(M, 16, omega=omega.to(device), granularity="per_row", debug=True)
    Mf = M.float()
    err = (torch.linalg.matrix_norm(Mf - torch.matmul(res["coeffs"], res["vh"])) / torch.linalg.matrix_norm(Mf))
    return M, omega, {"blocks_per_s": round(8 / (ms * 1e-3), 1), "ms_per_call": round(ms, 4), "batch": 8,
                      "k": 16, "oversampling": 5, "n_iter": 2, "quant": "per_row",
                      "layer_blocks_per_s": round(8 / (ms * 1e-3) / (2 * HKV), 1),
                      "gemm_flops_per_block": gemm_flops,
                      "mfma_fp16_utilisation": round(8 * gemm_flops / (ms * 1e-3) / (MFMA_FP16_PEAK_TFLOPS * 1e12), 6),
                      "recon_err": round(err.mean().item(), 6)}


def cpu_rsvd_baseline(M_gpu, omega):
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    sys.path.insert(0, HERE)
    from oracle.quant import quantize_per_row
    from oracle.rsvd import randomized_svd_ref
    M = M_gpu.cpu().numpy()
    rng = np.random.default_rng(8)
    cores = len(os.sched_getaffinity(0))
    with threadpool_limits(cores):
        blas = [i.get("num_threads") for i in threadpool_info()]
        times = []
        for _ in range(250):
            om = rng.standard_normal((8, D, 21)).astype(np.float32)
            t0 = time.perf_counter()
            U, S, Vh = randomized_svd_ref(M, 16, om)
            quantize_per_row(U * S[:, None, :])
            times.append(time.perf_counter() - t0)
        best = sorted(times)[len(times) // 2]
        U, S, Vh = randomized_svd_ref(M, 16, omega.numpy())
    Mf = M.astype(np.float64)
    err = np.linalg.norm(Mf - np.matmul(U * S[:, None, :], Vh), axis=(1, 2)) / np.linalg.norm(Mf, axis=(1, 2))
    return {"value": round(8 / best, 1), "unit": "blocks/s", "cores": max(b for b in blas if b) if blas else 1,
            "kind": "port", "recon_err": round(float(err.mean()), 6),
            "sample": "oracle randomized_svd_ref (float32 LAPACK restatement of rsvd.py) + "
                      f"per-row quantise, 8x512x128, k=16; median of 250 calls with fresh sketches "
                      f"({best * 1e3:.2f} ms, {sum(times):.1f} s in all)"}


def time_decode(torch, lib, hip, caches, Q, cos, sin, qpos, warmup, steps, split=0):
    """Warm-up calls, then `steps` calls issued back to back between two HIP
    events on the launch stream (the host enqueues ahead of the GPU, so the
    events measure the GPU time of the calls), then `steps` more calls each
    bracketed by its own events (isolated latency: includes the host's launch
    latency whenever the queue runs dry).  The tier sets in `caches` are used
    in rotation.  Returns (ms of the back-to-back loop, sorted isolated ms)."""
    from unsloth_spectral import _lib
    b = Q.shape[0]
    outs = [torch.empty(b, HQ, D, dtype=torch.float16, device=Q.device) for _ in caches]
    built = [decode_args(_lib, c, Q, o, cos, sin, qpos, split) for c, o in zip(caches, outs)]
    nbytes = ctypes.c_size_t(0)
    _lib.check(lib.sc_decode_workspace_size(ctypes.byref(built[0][0]), ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=Q.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(i):
        _lib.check(lib.sc_decode_attn(ctypes.byref(built[i % len(built)][0]), ctypes.c_void_p(ws.data_ptr()),
                                      ws.numel(), stream))

    for i in range(warmup):
        step(i)
    starts = [hip.event() for _ in range(steps)]
    ends = [hip.event() for _ in range(steps)]
    t0, t1 = hip.event(), hip.event()
    torch.cuda.synchronize()
    hip.record(t0, stream)
    for i in range(steps):
        step(i)
    hip.record(t1, stream)
    torch.cuda.synchronize()
    total_ms = hip.elapsed_ms(t0, t1)
    for i in range(steps):
        hip.record(starts[i], stream)
        step(i)
        hip.record(ends[i], stream)
    torch.cuda.synchronize()
    return total_ms, sorted(hip.elapsed_ms(a, e) for a, e in zip(starts, ends))


def compression_stall(torch, hip, cache_full, raw, reps=5):
    """Stall of one block compression inside a decode step (batch 16 x 8 KV
    heads, K and V: 256 rSVDs + quantisation in one launch).  A step is
    append(one token per sequence) + decode attention, event-timed on the
    stream; the compressing step starts from 511 tail tokens (the appended
    token completes a block), the plain step from 510."""
    from unsloth_spectral._decode import run_decode
    b, nb = cache_full._B, cache_full.num_cold_blocks
    cold = nb * TB
    Kx, Vx = raw
    cos, sin = rope_tables(torch, cold + 2 * TB, Kx.device)
    g = torch.Generator(device=Kx.device)
    g.manual_seed(11)
    Q = torch.randn(b, HQ, 1, D, generator=g, device=Kx.device).half()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    from unsloth_spectral import _lib

    def with_tail(n):  # the first n tail tokens of cache_full (tail ring head at slot 0)
        c = cache_full.clone()
        c._tail_len = n
        c.counters[:, _lib.SC_CNT_TAIL_LEN].fill_(n)
        c.counters[:, _lib.SC_CNT_NEXT_POS].fill_(cold + n)
        c.counters[:, _lib.SC_CNT_TOTAL].fill_(cold + n)
        c.total_tokens = c.current_position = cold + n
        return c

    times = {}
    for n in (510, 511) * (reps + 1):
        c = with_tail(n)
        k1 = Kx[:, cold + n:cold + n + 1].reshape(b, HKV, 1, D)
        v1 = Vx[:, cold + n:cold + n + 1].reshape(b, HKV, 1, D)
        torch.cuda.synchronize()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        c.append(k1, v1)
        run_decode(Q, c, cos, sin, cold + n, rope_mode=_lib.SC_ROPE_ABSOLUTE, halves_equal=True)
        hip.record(e1, stream)
        ms = hip.elapsed_ms(e0, e1)
        assert c.num_cold_blocks == nb + (n == 511)
        times.setdefault(n, []).append(ms)
        del c
    med = {n: sorted(v[1:])[len(v[1:]) // 2] for n, v in times.items()}
    return {"step_us_plain": round(med[510] * 1e3, 1), "step_us_compress": round(med[511] * 1e3, 1),
            "stall_us": round((med[511] - med[510]) * 1e3, 1), "matrices_per_compression": 2 * b * HKV,
            "reps": reps}


def decode_config(torch, lib, hip, device, b, nblk, k, tail, rotate, warmup, steps, on_device=False,
                  stall=False, cpu_seqs=0):
    """One secondary decode workload: event-timed call duration and the HBM
    roofline fraction of its algorithmic bytes."""
    log(f"building batch {b}, {nblk} cold blocks k={k}")
    cache0, raw, _ = build_decode(torch, device, b, nblk, k, tail, on_device=on_device,
                                  max_blocks=nblk + 1 if stall else None)
    ctx = nblk * TB + tail
    caches = [cache0] + [cache0.clone() for _ in range(rotate - 1)]
    cos, sin = rope_tables(torch, ctx + 64, device)
    g = torch.Generator(device=device)
    g.manual_seed(1)
    Q = torch.randn(b, HQ, D, generator=g, device=device).half()
    total_ms, per_call = time_decode(torch, lib, hip, caches, Q, cos, sin, ctx - 1, warmup, steps)
    avg = total_ms / steps
    iso = sum(per_call) / len(per_call)
    nbytes = decode_bytes(b, HKV, nblk, k, k, tail)
    ach = nbytes / (avg * 1e-3) / 1e9
    res = {"batch": b, "context": ctx, "cold_blocks": nblk, "rank": k, "tail": tail, "tier_sets_rotated": rotate,
           "steps": steps, "warmup": warmup, "us_per_layer": round(avg * 1e3, 2),
           "us_per_layer_isolated_call": round(iso * 1e3, 2),
           "us_per_layer_isolated_call_median": round(per_call[len(per_call) // 2] * 1e3, 2),
           "algorithmic_bytes_per_call": nbytes,
           "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4)}}
    del caches
    log(f"batch {b}: {avg * 1e3:.2f} us per call")
    if cpu_seqs:
        log(f"CPU baselines (oracle), {cpu_seqs} sequence(s) of batch {b}, both RoPE modes")
        res["cpu_baseline"] = {m: cpu_decode_baseline(cache0, Q, cos, sin, m, seqs=cpu_seqs)
                               for m in ("absolute", "distance")}
    if stall:
        res["compression_stall"] = compression_stall(torch, hip, cache0, raw)
        log(f"compression stall: {res['compression_stall']}")
    del cache0, raw
    torch.cuda.empty_cache()
    return res


def model_loop(torch, device, prompt, decode_steps, layers=32):
    """Mistral-7B-shaped transformers model (random FP16 weights): prefill of
    `prompt` tokens, then `decode_steps` greedy one-token steps, with the
    spectral cache (patch_unsloth_attention, k=16) and, on the same weights,
    with transformers' dense FP16 KV cache.  Tokens/s of the decode phase."""
    from transformers import MistralConfig, MistralForCausalLM
    from unsloth_spectral import get_cache_stats, patch_unsloth_attention
    cfg = MistralConfig(vocab_size=32768, hidden_size=4096, intermediate_size=14336, num_hidden_layers=layers,
                        num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                        max_position_embeddings=32768, rope_theta=1e6, sliding_window=None, rms_norm_eps=1e-5)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    t0 = time.perf_counter()
    with torch.device(device):
        model = MistralForCausalLM._from_config(cfg, dtype=torch.float16).eval()
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    log(f"model built in {init_s:.1f} s")
    g = torch.Generator().manual_seed(12)
    ids = torch.randint(0, cfg.vocab_size, (1, prompt), generator=g).to(device)

    def timed(fn):
        torch.cuda.synchronize()
        t = time.perf_counter()
        r = fn()
        torch.cuda.synchronize()
        return r, time.perf_counter() - t

    @torch.no_grad()
    def dense_run(n_prompt, steps):
        out = model(input_ids=ids[:, :n_prompt], use_cache=True, logits_to_keep=1)
        past, tok = out.past_key_values, out.logits[:, -1].argmax(-1)
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            out = model(input_ids=tok[:, None], past_key_values=past, use_cache=True, logits_to_keep=1)
            past, tok = out.past_key_values, out.logits[:, -1].argmax(-1)
        torch.cuda.synchronize()
        return time.perf_counter() - t

    @torch.no_grad()
    def spectral_run(n_prompt, steps):
        for layer in model.model.layers:
            layer.self_attn._spectral_cache = None
        out, pre_s = timed(lambda: model(input_ids=ids[:, :n_prompt], use_cache=False, logits_to_keep=1))
        tok = out.logits[:, -1].argmax(-1)
        pos_all = torch.arange(n_prompt, n_prompt + steps, device=device)[None]   # positions stay on the device
        toks = []
        torch.cuda.synchronize()
        t = time.perf_counter()
        for i in range(steps):
            out = model(input_ids=tok[:, None], position_ids=pos_all[:, i:i + 1], use_cache=False,
                        logits_to_keep=1)
            tok = out.logits[:, -1].argmax(-1)
            toks.append(tok)
        host_s = time.perf_counter() - t          # the host issued every step without waiting
        torch.cuda.synchronize()
        return pre_s, time.perf_counter() - t, host_s, torch.cat(toks)

    @torch.no_grad()
    def graph_run(n_prompt, steps):
        """The same greedy steps replayed from HIP graphs (CapturedDecode): one
        captured segment per stretch between block boundaries; the step that
        crosses a boundary (its append compresses) runs eagerly."""
        from unsloth_spectral import CapturedDecode
        for layer in model.model.layers:
            layer.self_attn._spectral_cache = None
        out = model(input_ids=ids[:, :n_prompt], use_cache=False, logits_to_keep=1)
        tok = out.logits[:, -1].argmax(-1)
        pos = torch.full((1, 1), n_prompt, dtype=torch.long, device=device)
        toks, done, segments = [], 0, 0
        torch.cuda.synchronize()
        t = time.perf_counter()
        while done < steps:
            tail = model.model.layers[0].self_attn._spectral_cache.hot_len
            seg = min(steps - done, TB - 1 - tail)
            if seg >= 3:
                dec = CapturedDecode(model, seg)
                segments += 1
                for _ in range(seg):
                    tok = dec.step(tok, pos).argmax(-1)
                    pos += 1
                    toks.append(tok)
            else:
                seg = max(seg, 1)
                for _ in range(seg):
                    out = model(input_ids=tok[:, None], position_ids=pos, use_cache=False, logits_to_keep=1)
                    tok = out.logits[:, -1].argmax(-1)
                    pos += 1
                    toks.append(tok)
            done += seg
        torch.cuda.synchronize()
        return time.perf_counter() - t, torch.cat(toks), segments

    dense_run(min(prompt, 1024), 4)                      # warm-up (kernels, allocator)
    dense_s = dense_run(prompt, decode_steps)
    log(f"dense KV cache: {dense_s / decode_steps * 1e3:.2f} ms per token")
    torch.cuda.empty_cache()
    patch_unsloth_attention(model, k_rank_keys=16, k_rank_values=16, verbose=False, quant_granularity="per_row")
    spectral_run(min(prompt, 1024) + 8, 4)
    prefill_s, spec_s, host_s, spec_tok = spectral_run(prompt, decode_steps)
    log(f"spectral cache: {spec_s / decode_steps * 1e3:.2f} ms per token, prefill {prefill_s:.2f} s")
    st = get_cache_stats(model)
    graph_run(min(prompt, 1024) + 8, 8)                   # warm-up of the captured path
    graph_s, graph_tok, graph_segments = graph_run(prompt, decode_steps)
    same = (graph_tok == spec_tok).float().mean().item()
    log(f"spectral cache, graph-replayed steps: {graph_s / decode_steps * 1e3:.2f} ms per token "
        f"({graph_segments} captured segments), same tokens as the eager steps: {same:.3f}")
    # decode attention of one token over every layer's final cache (HIP events)
    from unsloth_spectral import _lib
    from unsloth_spectral._decode import run_decode
    hip = Hip()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device=device)
    g.manual_seed(14)
    q1 = torch.randn(1, 32, 1, 128, generator=g, device=device).half()
    calls = []
    for layer in model.model.layers:
        attn = layer.self_attn
        c = attn._spectral_cache
        cos, sin = attn._spectral_rope.get(c.current_position + 1, device)
        calls.append((c, cos, sin, c.current_position - 1))
    for c, cos, sin, qp in calls:
        run_decode(q1, c, cos, sin, qp, rope_mode=_lib.SC_ROPE_ABSOLUTE, halves_equal=True)
    torch.cuda.synchronize()
    e0, e1 = hip.event(), hip.event()
    reps = 20
    hip.record(e0, stream)
    for _ in range(reps):
        for c, cos, sin, qp in calls:
            run_decode(q1, c, cos, sin, qp, rope_mode=_lib.SC_ROPE_ABSOLUTE, halves_equal=True)
    hip.record(e1, stream)
    attn_ms = hip.elapsed_ms(e0, e1) / reps
    return {
        "metric": "model decode tokens/s (spectral cache vs dense fp16 KV cache)",
        "value": round(decode_steps / spec_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": decode_steps,
        "warmup": 4, "ms_per_step": round(spec_s / decode_steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"transformers MistralForCausalLM, Mistral-7B shape ({layers} layers, hidden 4096, "
                               "32/8 heads, head_dim 128, FFN 14336, vocab 32768), random fp16 weights; "
                               f"{prompt}-token prompt + {decode_steps} greedy steps, batch 1; spectral cache k=16 "
                               "(K and V), per-row INT8 scales, absolute RoPE theta 1e6",
                   "prompt": prompt, "decode_steps": decode_steps, "layers": layers},
        "spectral": {"decode_ms_per_token": round(spec_s / decode_steps * 1e3, 3),
                     "host_issue_ms_per_token": round(host_s / decode_steps * 1e3, 3),
                     "prefill_s": round(prefill_s, 3),
                     "cold_blocks_per_layer": st["total_blocks"] // layers,
                     "compressions_during_decode": (prompt + decode_steps) // TB - prompt // TB,
                     "kv_bytes": st["total_compressed_bytes"], "kv_bytes_fp16": st["total_original_bytes"],
                     "compression_ratio": round(st["compression_ratio"], 3),
                     "attention_ms_per_token": round(attn_ms, 3),
                     "attention_share": round(attn_ms / (spec_s / decode_steps * 1e3), 4)},
        "spectral_graph_replay": {"decode_ms_per_token": round(graph_s / decode_steps * 1e3, 3),
                                  "tokens_per_s": round(decode_steps / graph_s, 2),
                                  "captured_segments": graph_segments,
                                  "same_tokens_as_eager_fraction": round(same, 4),
                                  "note": "unsloth_spectral.CapturedDecode: each stretch of steps between "
                                          "block boundaries captured once (the capture is inside the timed "
                                          "region) and replayed; greedy argmax between replays"},
        "dense_fp16_kv": {"decode_ms_per_token": round(dense_s / decode_steps * 1e3, 3),
                          "tokens_per_s": round(decode_steps / dense_s, 2)},
        "model_init_s": round(init_s, 1),
    }


def bench_block_pack(torch, hip, cache, reps=20):
    """sc_tier_pack of every cold block of every sequence (one launch per
    sequence), then sc_tier_unpack of the records back into the same slots;
    HBM bytes = each byte read once and written once."""
    B, nb = cache._B, cache.num_cold_blocks
    rb = cache.block_record_bytes()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    recs = [cache.export_blocks(b) for b in range(B)]
    torch.cuda.synchronize()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(reps):
        for b in range(B):
            cache.export_blocks(b)
    hip.record(e1, stream)
    pack_ms = hip.elapsed_ms(e0, e1) / reps
    hip.record(e0, stream)
    for _ in range(reps):
        for b in range(B):
            cache.import_blocks(recs[b], seq=b, first=0)
    hip.record(e1, stream)
    unpack_ms = hip.elapsed_ms(e0, e1) / reps
    total = B * nb * rb
    return {"records": B * nb, "record_bytes": rb, "pack_us": round(pack_ms * 1e3, 1),
            "pack_gbs": round(2 * total / (pack_ms * 1e-3) / 1e9, 1),
            "unpack_us_incl_status_read": round(unpack_ms * 1e3, 1),
            "unpack_gbs_incl_status_read": round(2 * total / (unpack_ms * 1e-3) / 1e9, 1),
            "note": "pack: one launch per sequence; unpack: header check + copy + a host read of the status "
                    "word per sequence (a synchronisation), so it is a lower bound on the kernels' rate"}


def bench_prefill(torch, hip, device, ctx=8192, k=16, reps=5):
    """One layer's prefill attention of a ctx-token prompt (batch 1, 32/8
    heads, causal) over its spectral tiers (ctx / 512 cold blocks of rank
    k): the HIP prefill kernel against the dense reference path (get_kv,
    apply_rope, fp16 attention in 1024-row slices)."""
    from unsloth_spectral._prefill import run_prefill
    from unsloth_spectral.integration import _dense_prefill
    nblk = ctx // TB
    cache, raw, _ = build_decode(torch, device, 1, nblk, k, 0, on_device=True)
    del raw
    cos, sin = rope_tables(torch, ctx + 64, device)
    g = torch.Generator(device=device)
    g.manual_seed(13)
    Q = torch.randn(1, HQ, ctx, D, generator=g, device=device).half()
    pos = torch.arange(ctx, device=device)[None]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        for _ in range(reps):
            out = fn()
        hip.record(e1, stream)
        return hip.elapsed_ms(e0, e1) / reps, out

    ms_k, out_k = timed(lambda: run_prefill(Q, cache, cos, sin, pos))
    ms_d, out_d = timed(lambda: _dense_prefill(Q, cache, cos, sin, HQ // HKV, None, 1.0 / math.sqrt(D), pos))
    err = (out_k.float() - out_d.float()).abs().max().item()
    flops = 2 * 2 * HQ * D * ctx * (ctx + 1) / 2  # causal QK^T and PV
    return {"context": ctx, "cold_blocks": nblk, "rank": k, "batch": 1, "kernel_ms": round(ms_k, 3),
            "dense_reference_path_ms": round(ms_d, 3), "speedup": round(ms_d / ms_k, 2),
            "attention_tflops": round(flops / (ms_k * 1e-3) / 1e12, 1),
            "mfma_fp16_frac": round(flops / (ms_k * 1e-3) / (MFMA_FP16_PEAK_TFLOPS * 1e12), 4),
            "max_abs_diff_vs_dense": round(err, 5)}


TRAFFIC_JSON = os.path.join(HERE, "profiles", "decode_c3_traffic.json")


def load_traffic():
    if not os.path.exists(TRAFFIC_JSON):
        return None
    with open(TRAFFIC_JSON) as f:
        return json.load(f).get("hbm_bytes_per_call")


def copy_probe(torch, device, mib, reps=5):
    """A plain streaming kernel of known size for counter calibration:
    torch.neg over mib MiB of fp16 reads mib MiB and writes mib MiB."""
    src = torch.ones(mib << 19, dtype=torch.float16, device=device)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def _pmc_means(path):
    """Mean value per dispatch of every counter, per kernel name, from what a
    rocprofv3 --pmc run wrote under path (counter_collection CSV files, or
    rocpd databases)."""
    import collections
    import csv
    import glob
    import sqlite3
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for fn in glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True):
        with open(fn) as f:
            for r in csv.DictReader(f):
                agg[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    for db in glob.glob(os.path.join(path, "**", "*_results.db"), recursive=True):
        con = sqlite3.connect(db)
        cur = con.cursor()
        cols = [r[1] for r in cur.execute("pragma table_info(counters_collection)")]
        ci = {c: i for i, c in enumerate(cols)}
        name_k = "kernel_name" if "kernel_name" in ci else "name"
        for r in cur.execute("select * from counters_collection"):
            agg[r[ci[name_k]]][r[ci["counter_name"]]].append(r[ci["value"]])
        con.close()
    return {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in agg.items()}


def summarize_pmc(fetch_dir, write_dir, mib):
    """HBM traffic of one decode call from two rocprofv3 --pmc runs of this
    script (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by
    what the same counter reads for the copy probe of mib MiB."""
    fetch, write = _pmc_means(fetch_dir), _pmc_means(write_dir)

    def pick(tab, key, counter):
        vals = {k: v[counter] for k, v in tab.items() if key in k and counter in v}
        if not vals:
            raise SystemExit(f"no kernel matching {key!r} with {counter}")
        if len(vals) > 1:  # the largest dispatch is the one of interest (the copy probe)
            print(f"{len(vals)} kernels match {key!r}: " + "; ".join(f"{k[:90]} = {v:.1f}" for k, v in vals.items()),
                  file=sys.stderr)
        return max(vals.values())

    kib = mib * 1024.0
    f_copy, w_copy = pick(fetch, "neg_kernel", "FETCH_SIZE"), pick(write, "neg_kernel", "WRITE_SIZE")
    f_factor, w_factor = kib / f_copy, kib / w_copy
    parts = {}
    for key in ("decode_partial_kernel", "decode_combine_kernel"):
        f, w = pick(fetch, key, "FETCH_SIZE"), pick(write, key, "WRITE_SIZE")
        parts[key] = {"fetch_kib_raw": round(f, 1), "write_kib_raw": round(w, 1),
                      "hbm_bytes": int(round((f * f_factor + w * w_factor) * 1024))}
    total = sum(v["hbm_bytes"] for v in parts.values())
    nb = decode_bytes(B, HKV, NBLK, K_RANK, K_RANK, TAIL)
    out = {"hbm_bytes_per_call": total, "algorithmic_bytes_per_call": nb,
           "traffic_over_algorithmic": round(total / nb, 4), "kernels": parts,
           "copy_probe": {"mib": mib, "fetch_kib_raw": round(f_copy, 1), "write_kib_raw": round(w_copy, 1),
                          "fetch_factor": round(f_factor, 5), "write_factor": round(w_factor, 5)}}
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=3000)  # ~0.15 s: GPU clocks settle before timing
    ap.add_argument("--rotate", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-headline", action="store_true",
                    help="time only the batch-8 decode workload and the rSVD (profiling runs)")
    ap.add_argument("--model-loop", action="store_true",
                    help="run only the Mistral-7B-shaped model loop and print its JSON line")
    ap.add_argument("--no-model-loop", action="store_true",
                    help="leave the model loop out of the default line (profiling runs)")
    ap.add_argument("--split", type=int, default=0,
                    help="workgroups per cold block for the batch-8 workload (0 = library's choice)")
    ap.add_argument("--prompt", type=int, default=8192)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain copy kernel of this size first (counter calibration)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write the decode traffic JSON from two rocprofv3 --pmc runs and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc, args.copy_probe_mib)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the spectral decode path has no "
                                   "multi-GPU collective; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from unsloth_spectral import _lib
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    lib = _lib.load()
    hip = Hip()
    if args.model_loop:
        print(json.dumps(model_loop(torch, device, args.prompt, args.decode_steps)))
        return
    if args.copy_probe_mib:
        copy_probe(torch, device, args.copy_probe_mib)

    log("building the batch-8 16K tiers")
    cache0, raw = build_c3(torch, device)
    del raw
    log("timing decode, batch 8")
    caches = [cache0] + [cache0.clone() for _ in range(args.rotate - 1)]
    cos, sin = rope_tables(torch, CTX + 64, device)
    g = torch.Generator(device=device)
    g.manual_seed(1)
    Q = torch.randn(B, HQ, D, generator=g, device=device).half()
    total_ms, per_call = time_decode(torch, lib, hip, caches, Q, cos, sin, CTX - 1, args.warmup, args.steps,
                                     args.split)
    iso_call_ms = sum(per_call) / len(per_call)
    med_call_ms = per_call[len(per_call) // 2]
    ms_per_step = total_ms / args.steps
    nb = decode_bytes(B, HKV, NBLK, K_RANK, K_RANK, TAIL)
    rope_bytes = CTX * (D // 2) * 2 * 2
    achieved = nb / (ms_per_step * 1e-3) / 1e9
    traffic = load_traffic()

    log(f"decode batch 8: {ms_per_step * 1e3:.2f} us per call back to back, {iso_call_ms * 1e3:.2f} us isolated; "
        "timing rSVD")
    M_rsvd, omega, rsvd = bench_rsvd(torch, hip, device)
    cpu = cpu_rsvd = None
    cpu_dist = None
    if not args.no_cpu:
        log("CPU baselines (oracle), batch 8: absolute and distance RoPE")
        cpu = cpu_decode_baseline(cache0, Q.view(B, HQ, D), cos, sin)
        cpu_dist = cpu_decode_baseline(cache0, Q.view(B, HQ, D), cos, sin, "distance")
        cpu_rsvd = cpu_rsvd_baseline(M_rsvd, omega)
        rsvd["cpu_baseline"] = cpu_rsvd
        rsvd["recon_err_rel_diff_vs_oracle"] = round(abs(rsvd["recon_err"] - cpu_rsvd["recon_err"])
                                                     / cpu_rsvd["recon_err"], 5)
        rsvd["rank32_parity"] = rsvd_rank32_parity(torch, M_rsvd)
    others = None
    if not args.only_headline:
        log("block wire format: pack / unpack of the batch-8 tiers")
        wire = bench_block_pack(torch, hip, cache0)
        del caches, cache0
        torch.cuda.empty_cache()
        log("decode batch 1 (4K) and batch 16 (33K, with compression stall)")
        others = {
            "batch1_ctx4096": decode_config(torch, lib, hip, device, 1, 7, 16, 512, args.rotate, 1000, 200,
                                            cpu_seqs=0 if args.no_cpu else 1),
            "batch16_ctx33280": decode_config(torch, lib, hip, device, 16, 64, 32, 512, 2, 300, 100,
                                              on_device=True, stall=True, cpu_seqs=0 if args.no_cpu else 2),
            "block_wire_format": wire,
        }
        log("prefill attention, 8192-token prompt over 16 cold blocks")
        others["prefill_ctx8192"] = bench_prefill(torch, hip, device)
        if not args.no_model_loop:
            torch.cuda.empty_cache()
            log("model loop: Mistral-7B shape, 8192-token prompt + 256 greedy steps")
            others["model_loop"] = model_loop(torch, device, args.prompt, args.decode_steps)
    res = {
        "metric": "decode attn µs/layer + HBM GB/s (% peak) at 16K ctx; rSVD blocks/sec",
        "value": round(nb / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "spectral decode attention, one layer: batch 8, context 16384 (31 cold 512-token "
                               "blocks k=32 + 512 fp16 tail), 32 q / 8 kv heads, head_dim 128, per-row INT8 scales, "
                               "absolute RoPE theta 1e6",
                   "batch": B, "context": CTX, "cold_blocks": NBLK, "rank": K_RANK, "tail": TAIL,
                   "tier_sets_rotated": args.rotate},
        "us_per_layer": round(ms_per_step * 1e3, 2),
        "us_per_layer_isolated_call": round(iso_call_ms * 1e3, 2),
        "us_per_layer_isolated_call_median": round(med_call_ms * 1e3, 2),
        "algorithmic_bytes_per_call": nb,
        "rope_table_bytes_half_rows": rope_bytes,
        "hbm_peak_fraction_of_value": round(nb / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "sc_decode_attn call (decode_partial_kernel + decode_combine_kernel)"},
        "cpu_baseline": cpu,
        "cpu_baseline_distance_rope": cpu_dist,
        "rsvd": rsvd,
        "other_decode_workloads": others,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
