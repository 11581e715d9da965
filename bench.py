"""Benchmark: spectral decode attention (C3) + rSVD block compression (C2) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--rotate R]
    python bench.py ... --copy-probe-mib 256          (under rocprofv3 --pmc: calibration kernel)
    python bench.py --summarize-pmc FETCH_DIR WRITE_DIR --copy-probe-mib 256

Workloads (synthetic data, seeds fixed):
  decode  batch 8, context 16384 = 31 cold 512-token blocks (INT8 codes k=32,
          one FP32 scale per row, FP16 bases) + 512 FP16 tail tokens per
          sequence; 32 query / 8 KV heads, head_dim 128, absolute RoPE
          (theta 1e6).  K/V are U diag(exp(-i/8)) V^T + N(0, 0.01^2) per
          (sequence, KV head); the cold blocks are compressed on the GPU by
          this library's rSVD (k=32, p=5, q=2) before timing.  One step = one
          decode-attention call for one layer.  R distinct tier sets (default
          4, ~490 MB of tiers) are rotated so that the 256 MB MALL cannot hold
          the working set.
  rsvd    8 x 512 x 128 FP16 blocks of the same distribution, k=16, p=5, q=2,
          per-row INT8 quantisation; blocks/sec = matrices per second.
Prints one JSON line.  value = algorithmic HBM bytes of one decode call
divided by the measured time per step (GB/s); roofline.achieved uses the
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
FP32_VALU_PEAK_TFLOPS = 78.6  # non-packed FP32 vector (packed FP32 is disabled in these kernels)

B, HQ, HKV, D, TB, NBLK, K_RANK, TAIL = 8, 32, 8, 128, 512, 31, 32, 512
CTX = NBLK * TB + TAIL


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


def build_c3(torch, device):
    """Tier state of the decode workload, compressed by the HIP rSVD."""
    from unsloth_spectral import SpectralCache, compress_matrices
    Kx = lowrank_kv(torch, 2, B * HKV, CTX, D, device)
    Vx = lowrank_kv(torch, 3, B * HKV, CTX, D, device)
    cold = NBLK * TB
    tiers = []
    for X, seed in ((Kx, 4), (Vx, 5)):
        M = X[:, :cold].reshape(B * HKV * NBLK, TB, D)
        r = compress_matrices(M, K_RANK, seed=seed, granularity="per_row")
        tiers.append((r["codes"].view(B, HKV, NBLK, TB, -1)[..., :K_RANK],
                      r["scales"].view(B, HKV, NBLK, TB),
                      r["basis"].view(B, HKV, NBLK, -1, D)[:, :, :, :K_RANK],
                      r["minmax"].view(B, HKV, NBLK, 2)))
    (ck, sk, bk, mk), (cv, sv, bv, mv) = tiers
    start = (torch.arange(NBLK, device=device) * TB)[None].expand(B, NBLK)
    tk = Kx[:, cold:].reshape(B, HKV, TAIL, D)
    tv = Vx[:, cold:].reshape(B, HKV, TAIL, D)
    tp = torch.arange(cold, CTX, device=device)[None].expand(B, TAIL)
    cache = SpectralCache.from_tiers(ck, sk, bk, cv, sv, bv, start, tk, tv, tp, block_size=TB,
                                     tail_capacity=2 * TB, minmax_k=mk, minmax_v=mv)
    return cache, (Kx, Vx)


def rope_tables(torch, length, device, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=device, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(length, device=device, dtype=torch.float32), inv)
    emb = torch.cat([emb, emb], dim=-1)
    return emb.cos().half().contiguous(), emb.sin().half().contiguous()


def decode_args(lib_mod, cache, Q, out, cos, sin, qpos):
    a = lib_mod.ScDecodeArgs()
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


def cpu_decode_baseline(cache, Q, cos, sin):
    """The oracle (fp16-faithful restatement of spectral_attention_decode) on
    sequence 0 of the same workload, timed on the host cores."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    sys.path.insert(0, HERE)
    from oracle.attention import ColdBlock, TierState, spectral_attention_decode
    cores = len(os.sched_getaffinity(0))
    nb = cache.num_cold_blocks
    ck = cache.codes_k[0, :, :nb, :, :K_RANK].cpu().numpy()
    cv = cache.codes_v[0, :, :nb, :K_RANK, :].transpose(-1, -2).cpu().numpy()
    sk = cache.scales_k[0, :, :nb].cpu().numpy()
    sv = cache.scales_v[0, :, :nb].cpu().numpy()
    bk = cache.basis_k[0, :, :nb, :, :K_RANK].transpose(-1, -2).cpu().numpy()
    bv = cache.basis_v[0, :, :nb, :, :K_RANK].transpose(-1, -2).cpu().numpy()
    blocks = [ColdBlock(ck[:, j], sk[:, j], bk[:, j], cv[:, j], sv[:, j], bv[:, j], j * TB) for j in range(nb)]
    st = TierState(blocks, cache.hot_K[0].cpu().numpy(), cache.hot_V[0].cpu().numpy(),
                   cache.hot_position_ids[0].cpu().numpy())
    q = Q[0].cpu().numpy()
    c, s = cos.cpu().numpy(), sin.cpu().numpy()
    with threadpool_limits(cores):
        blas = [i.get("num_threads") for i in threadpool_info()]
        t0 = time.perf_counter()
        spectral_attention_decode(q, st, c, s, CTX - 1)
        t1 = time.perf_counter()
        spectral_attention_decode(q, st, c, s, CTX - 1)
        t2 = time.perf_counter()
    sec = min(t1 - t0, t2 - t1)
    seq_bytes = decode_bytes(1, HKV, NBLK, K_RANK, K_RANK, TAIL)
    return {"value": round(seq_bytes / sec / 1e9, 4), "unit": "GB/s", "cores": max(b for b in blas if b) if blas else 1,
            "kind": "port", "us_per_layer_batch8": round(sec * 8 * 1e6, 1),
            "sample": "oracle spectral_attention_decode (fp16-faithful numpy restatement), sequence 0 of 8, "
                      f"absolute RoPE, best of 2 runs ({sec:.2f} s each); the batch runs as 8 independent "
                      "batch-1 caches, so us_per_layer_batch8 = 8 x one sequence"}


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
    return M, {"blocks_per_s": round(8 / (ms * 1e-3), 1), "ms_per_call": round(ms, 4), "batch": 8,
               "k": 16, "oversampling": 5, "n_iter": 2, "quant": "per_row",
               "gemm_flops_per_block": gemm_flops,
               "valu_fp32_utilisation": round(8 * gemm_flops / (ms * 1e-3) / (FP32_VALU_PEAK_TFLOPS * 1e12), 5)}


def cpu_rsvd_baseline(M_gpu):
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
        best = 1e9
        for _ in range(5):
            om = rng.standard_normal((8, D, 21)).astype(np.float32)
            t0 = time.perf_counter()
            U, S, Vh = randomized_svd_ref(M, 16, om)
            quantize_per_row(U * S[:, None, :])
            best = min(best, time.perf_counter() - t0)
    return {"value": round(8 / best, 1), "unit": "blocks/s", "cores": max(b for b in blas if b) if blas else 1,
            "kind": "port", "sample": "oracle randomized_svd_ref (float32 LAPACK restatement of rsvd.py) + "
                                      f"per-row quantise, 8x512x128, k=16; best of 5 ({best * 1e3:.2f} ms)"}


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
    if args.copy_probe_mib:
        copy_probe(torch, device, args.copy_probe_mib)

    cache0, raw = build_c3(torch, device)
    del raw
    caches = [cache0] + [cache0.clone() for _ in range(args.rotate - 1)]
    cos, sin = rope_tables(torch, CTX + 64, device)
    g = torch.Generator(device=device)
    g.manual_seed(1)
    Q = torch.randn(B, HQ, D, generator=g, device=device).half()
    outs = [torch.empty(B, HQ, D, dtype=torch.float16, device=device) for _ in caches]
    built = [decode_args(_lib, c, Q, o, cos, sin, CTX - 1) for c, o in zip(caches, outs)]
    nbytes = ctypes.c_size_t(0)
    _lib.check(lib.sc_decode_workspace_size(ctypes.byref(built[0][0]), ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step(i):
        _lib.check(lib.sc_decode_attn(ctypes.byref(built[i % len(built)][0]), ctypes.c_void_p(ws.data_ptr()),
                                      ws.numel(), stream))

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    starts = [hip.event() for _ in range(args.steps)]
    ends = [hip.event() for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        hip.record(starts[i], stream)
        step(i)
        hip.record(ends[i], stream)
    torch.cuda.synchronize()
    total_ms = hip.elapsed_ms(starts[0], ends[-1])
    per_call = sorted(hip.elapsed_ms(s, e) for s, e in zip(starts, ends))
    avg_call_ms = sum(per_call) / len(per_call)
    med_call_ms = per_call[len(per_call) // 2]
    ms_per_step = total_ms / args.steps
    nb = decode_bytes(B, HKV, NBLK, K_RANK, K_RANK, TAIL)
    rope_bytes = CTX * (D // 2) * 2 * 2
    achieved = nb / (avg_call_ms * 1e-3) / 1e9
    traffic = load_traffic()

    M_rsvd, rsvd = bench_rsvd(torch, hip, device)
    cpu = cpu_rsvd = None
    if not args.no_cpu:
        cpu = cpu_decode_baseline(cache0, Q.view(B, HQ, D), cos, sin)
        cpu_rsvd = cpu_rsvd_baseline(M_rsvd)
        rsvd["cpu_baseline"] = cpu_rsvd
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
        "us_per_layer": round(avg_call_ms * 1e3, 2),
        "us_per_layer_median": round(med_call_ms * 1e3, 2),
        "algorithmic_bytes_per_call": nb,
        "rope_table_bytes_half_rows": rope_bytes,
        "hbm_peak_fraction_of_value": round(nb / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "sc_decode_attn call (decode_partial_kernel + decode_combine_kernel)"},
        "cpu_baseline": cpu,
        "rsvd": rsvd,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
