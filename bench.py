"""Benchmark of the FP8 quantized inference hot path on one MI355X.

One step of the hot path = the three kernels BASELINE names, each on its own
synthetic workload with inputs resident in HBM:
  * FP8 linear at the north-star shape [10800 x 3072] x [3072 x 12288]
    (per-token activation quant + row/col-scaled FP8 GEMM with bias, GELU-tanh)
  * FP8 KV quantize-on-write, config 2: K, V [1, 24, 10800, 128]
  * FP8-KV chunk attention, config 3: Q [1, 24, 10800, 128] over 86400 cached tokens
``value`` is the FP8 linear's TFLOP/s (the metric's headline); the attention
ms / GB/s and the KV-write GB/s ride along in the same JSON line, as does the
config-1 linear. Timing uses HIP events on the stream the kernels run on.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--only all|linear|kv|attn|copy]
``--only`` runs one workload (for per-kernel counter passes); ``copy`` is a
plain 1 GiB device copy used to calibrate the FETCH_SIZE / WRITE_SIZE counters.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP8_PEAK_TFLOPS = 5000.0     # MI355X dense FP8 MFMA
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense BF16 MFMA
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E

# Workload shapes: the north-star linear, config 1, the config-2 KV write and
# the config-3 attention (Q of the last chunk over 8 cached chunks).
NS_M, NS_K, NS_N = 10800, 3072, 12288
C1_M, C1_K, C1_N = 4096, 3072, 3072
KV_H, KV_L, KV_D = 24, 10800, 128
ATT_CHUNKS = 8
ATT_LQ, ATT_LK = KV_L, ATT_CHUNKS * KV_L   # config 3: 10800 queries over 86400 cached keys


def gemm_flops(m, k, n):
    return 2.0 * m * k * n


def kv_write_bytes(h=KV_H, l=KV_L, d=KV_D):
    rows = 2 * h * l                     # K and V rows
    return rows * d * 2 + rows * d + rows * 4   # bf16 in, e4m3 out, fp32 scale out


def attn_flops(h, lq, lk, d):
    return 4.0 * h * lq * lk * d


def attn_unique_bytes(h, lq, lk, d):
    return h * lq * d * 2 * 2 + 2 * h * lk * d + 2 * h * lk * 4   # Q + O bf16, K/V codes, scales


def time_loop(fn, steps, warmup, stream=None):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream() if stream is None else stream
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(s)
    for _ in range(steps):
        fn()
    end.record(s)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps   # ms per call


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 100 timed steps after 50 warmup steps: the north-star linear is ~0.4 ms,
    # and 20 steps after 5 warmup fell inside the clock transient of a GPU
    # coming out of idle (the same GEMM's calls drift from 410 to 510 us and
    # back within the first ~30 calls), reading 15 % low.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-ar", action="store_true", help="skip the config-5 AR chunk (about 15 s)")
    ap.add_argument("--only", default="all", choices=["all", "linear", "kv", "attn", "copy", "ar"])
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "sharding the hot path over several GPUs (heads for KV write and attention, tokens "
              "for the linear) is not built.", file=sys.stderr)
        sys.exit(2)

    import torch
    pkg = importlib.import_module("hy-nomas_amd")
    ops = pkg.ops
    kvc = importlib.import_module("hy-nomas_amd.fp8_kv_cache")
    ca = importlib.import_module("hy-nomas_amd.cache_attention")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if args.only == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        ms = time_loop(lambda: dst.copy_(src), args.steps, args.warmup)
        log(f"copy 1 GiB: {ms:.3f} ms ({2 * (1 << 30) / (ms * 1e-3) / 1e9:.0f} GB/s read+write)")
        return
    if args.only == "ar":
        print(json.dumps(bench_ar(args, torch, ops, dev, log)))
        return
    if args.only != "all":
        return run_only(args, torch, ops, kvc, ca, dev, log)

    # ---------------- FP8 linear, north-star shape
    g = torch.Generator(device=dev).manual_seed(1234)
    x = torch.randn(NS_M, NS_K, device=dev, generator=g)
    x = torch.where(torch.rand(NS_M, NS_K, device=dev, generator=g) < 0.001, x * 20, x).to(torch.bfloat16)
    w = (torch.randn(NS_N, NS_K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(NS_N, device=dev, generator=g) * 0.01).to(torch.bfloat16)
    qw, sw = ops.quantize_rows_fp8(w)
    del w
    qx, sx = ops.quantize_rows_fp8(x)

    ms_linear = time_loop(lambda: ops.linear_fp8(x, qw, sw, bias, 1), args.steps, args.warmup)
    ms_gemm = time_loop(lambda: ops.gemm_fp8_rowcol(qx, qw, sx, sw, bias, 1), args.steps, args.warmup)
    # The short kernels are timed through the C ABI with preallocated outputs:
    # at ~20 us per call, Python op dispatch would otherwise leave the GPU idle
    # between launches and the loop would time the host.
    L = importlib.import_module("hy-nomas_amd._lib")
    lib = L.load()
    qx_buf = torch.empty_like(qx)
    sx_buf = torch.empty_like(sx)
    stream_ptr = torch.cuda.current_stream().cuda_stream
    L.check(lib.hn_quantize_rows_fp8(x.data_ptr(), NS_M, NS_K, NS_K, L.HN_SCALE_CLAMP, 1e-4,
                                     qx_buf.data_ptr(), sx_buf.data_ptr(), stream_ptr),
            "hn_quantize_rows_fp8")
    ms_quant = time_loop(lambda: lib.hn_quantize_rows_fp8(
        x.data_ptr(), NS_M, NS_K, NS_K, L.HN_SCALE_CLAMP, 1e-4, qx_buf.data_ptr(),
        sx_buf.data_ptr(), stream_ptr), args.steps, args.warmup)
    f_ns = gemm_flops(NS_M, NS_K, NS_N)
    linear_tflops = f_ns / (ms_linear * 1e-3) / 1e12
    gemm_tflops = f_ns / (ms_gemm * 1e-3) / 1e12
    quant_bytes = NS_M * NS_K * 3 + NS_M * 4
    log(f"north-star linear {ms_linear:.3f} ms ({linear_tflops:.0f} TFLOP/s); "
        f"GEMM {ms_gemm:.3f} ms ({gemm_tflops:.0f} TFLOP/s); act quant {ms_quant * 1e3:.1f} us")
    del x, qx

    # ---------------- config 1 linear
    x1 = torch.randn(C1_M, C1_K, device=dev, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(C1_N, C1_K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    b1 = (torch.randn(C1_N, device=dev, generator=g) * 0.01).to(torch.bfloat16)
    qw1, sw1 = ops.quantize_rows_fp8(w1)
    ms_c1 = time_loop(lambda: ops.linear_fp8(x1, qw1, sw1, b1, 0), args.steps, args.warmup)
    c1_tflops = gemm_flops(C1_M, C1_K, C1_N) / (ms_c1 * 1e-3) / 1e12
    log(f"config-1 linear {ms_c1 * 1e3:.1f} us ({c1_tflops:.0f} TFLOP/s)")
    del x1, w1

    # ---------------- config 2: KV quantize-on-write
    gain = torch.empty(KV_H, device=dev).uniform_(0.5, 4.0, generator=g)
    k = (torch.randn(1, KV_H, KV_L, KV_D, device=dev, generator=g) * gain[None, :, None, None]).to(torch.bfloat16)
    v = (torch.randn(1, KV_H, KV_L, KV_D, device=dev, generator=g) * gain[None, :, None, None]).to(torch.bfloat16)
    cache = kvc.make_fp8_kv_block(1, ATT_CHUNKS * KV_L, KV_H, KV_D, device=dev)
    kt, vt = k.transpose(1, 2), v.transpose(1, 2)        # [1, L, H, D] views of BHSD data
    slot = (ATT_CHUNKS - 1) * KV_L
    kv_args = (L.HN_KV_FP8, kt.data_ptr(), vt.data_ptr(), L.strides(kt), 1, KV_L, KV_H, KV_D,
               cache["k"].data_ptr(), cache["v"].data_ptr(), L.strides(cache["k"]),
               cache["k_scale"].data_ptr(), cache["v_scale"].data_ptr(), L.strides(cache["k_scale"]),
               cache["k"].shape[1], slot, None, stream_ptr)
    L.check(lib.hn_kv_quantize_pair(*kv_args), "hn_kv_quantize_pair")
    ms_kv = time_loop(lambda: lib.hn_kv_quantize_pair(*kv_args), args.steps, args.warmup)
    kv_gbs = kv_write_bytes() / (ms_kv * 1e-3) / 1e9
    log(f"KV write {ms_kv * 1e3:.1f} us ({kv_gbs:.0f} GB/s)")

    # ---------------- config 3: chunk attention over 8 chunks
    for c in range(ATT_CHUNKS):
        gain = torch.empty(KV_H, device=dev).uniform_(0.5, 4.0, generator=g)
        kc = (torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
        vc = (torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
        kvc.quantize_kv_pair_into(cache, kc, vc, c * KV_L)
    del kc, vc, k, v
    q = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
    lk = ATT_CHUNKS * KV_L
    att_fn = lambda: ca.chunk_attention(q, cache, lk, q_pos0=(ATT_CHUNKS - 1) * KV_L, chunk_len=KV_L)
    ms_att = time_loop(att_fn, max(2, args.steps // 4), max(1, args.warmup // 2))
    att_tflops = attn_flops(KV_H, KV_L, lk, KV_D) / (ms_att * 1e-3) / 1e12
    att_gbs = attn_unique_bytes(KV_H, KV_L, lk, KV_D) / (ms_att * 1e-3) / 1e9
    log(f"chunk attention {ms_att:.3f} ms ({att_tflops:.0f} TFLOP/s, {att_gbs:.0f} GB/s unique)")
    # decode-style variant: 128 queries over the same cache (HBM-bound regime)
    qd = q[:, :128].contiguous()
    ms_dec = time_loop(lambda: ca.chunk_attention(qd, cache, lk), args.steps, args.warmup)
    dec_gbs = attn_unique_bytes(KV_H, 128, lk, KV_D) / (ms_dec * 1e-3) / 1e9
    log(f"decode-style attention (Lq=128) {ms_dec * 1e3:.1f} us ({dec_gbs:.0f} GB/s)")

    # ---------------- config 4: one FP8 DiT block over 7 cached chunks + the current one
    blk_res = bench_block(args, torch, cache, dev, g, log)
    del cache, q, qd

    # ---------------- config 5: 40-block AR chunk at the largest cache
    ar_res = bench_ar(args, torch, ops, dev, log) if not args.no_ar else None

    # ---------------- CPU baseline: the oracle's dequantize-then-matmul
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds, log)

    result = {
        "metric": "FP8 linear TFLOP/s (% MFMA peak); FP8-KV chunk attn ms + HBM GB/s",
        "value": round(linear_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_linear + ms_kv + ms_att, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 (fp32 accumulate); attention bf16 MFMA over e4m3 KV",
        "data": "synthetic (seeded N(0,1) activations with 0.1% x20 outliers, N(0,0.02) weights)",
        "config": {
            "workload": "north-star FP8 linear [10800x3072]x[3072x12288]+bias+GELU; "
                        "config-2 KV write; config-3 chunk attention (Lq 10800, Lk 86400, H 24, D 128)",
            "linear_mnk": [NS_M, NS_N, NS_K],
            "kv_write": [1, KV_H, KV_L, KV_D],
            "attention": {"Lq": KV_L, "Lk": lk, "H": KV_H, "D": KV_D, "chunk": KV_L},
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(gemm_tflops, 2),
            "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
            "traffic": gemm_traffic_bytes(),
        },
        "linear": {"ms": round(ms_linear, 4), "tflops": round(linear_tflops, 2),
                   "frac_fp8_peak": round(linear_tflops / FP8_PEAK_TFLOPS, 4),
                   "gemm_ms": round(ms_gemm, 4), "act_quant_us": round(ms_quant * 1e3, 2),
                   "act_quant_gbs": round(quant_bytes / (ms_quant * 1e-3) / 1e9, 1)},
        "config1_linear": {"us": round(ms_c1 * 1e3, 2), "tflops": round(c1_tflops, 2),
                           "frac_fp8_peak": round(c1_tflops / FP8_PEAK_TFLOPS, 4)},
        "kv_write": {"us": round(ms_kv * 1e3, 2), "gbs": round(kv_gbs, 1),
                     "frac_hbm": round(kv_gbs / HBM_PEAK_GBS, 4), "bytes": kv_write_bytes()},
        "attention": {"ms": round(ms_att, 4), "tflops": round(att_tflops, 2),
                      "frac_bf16_peak": round(att_tflops / BF16_PEAK_TFLOPS, 4),
                      "unique_hbm_gbs": round(att_gbs, 1),
                      "decode_lq128_us": round(ms_dec * 1e3, 2),
                      "decode_lq128_gbs": round(dec_gbs, 1),
                      "decode_frac_hbm": round(dec_gbs / HBM_PEAK_GBS, 4)},
        "dit_block": blk_res,
        "ar_chunk": ar_res,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))


def block_flops(hidden=3072, heads=24, tokens=KV_L, keys=ATT_CHUNKS * KV_L, d=KV_D, mlp=4):
    """Linears (QKV, out-proj, fc1, fc2) + attention over ``keys`` keys."""
    lin = 2.0 * tokens * hidden * (3 * hidden + hidden + 2 * mlp * hidden)
    return lin, attn_flops(heads, tokens, keys, d)


def bench_block(args, torch, cache, dev, g, log):
    """Config 4: one block's image stream, FP8 linears, attention over the FP8
    cache's first 7 chunks plus the current chunk as a bf16 tail."""
    db = importlib.import_module("hy-nomas_amd.dit_block")
    metrics = importlib.import_module("hy-nomas_amd.metrics")
    hist = (ATT_CHUNKS - 1) * KV_L
    blk = db.FP8DiTBlock(3072, KV_H, device=dev, generator=g)
    img = torch.randn(1, KV_L, 3072, device=dev, generator=g).to(torch.bfloat16)
    vec = torch.randn(1, 3072, device=dev, generator=g).to(torch.bfloat16)
    cos, sin = db.rope_tables(3, 45, 80, t_offset=3 * (ATT_CHUNKS - 1), device=dev)
    fn = lambda: blk(img, vec, cos, sin, cache, hist, update_cache=False)
    with torch.no_grad():
        ms = time_loop(fn, max(2, args.steps // 4), max(1, args.warmup // 2))
        with metrics.StageMetrics() as m:
            fn()
    lin, att = block_flops()
    tflops = (lin + att) / (ms * 1e-3) / 1e12
    stages = {k: round(v["seconds"] * 1e3, 3) for k, v in m.summary().items()}
    log(f"config-4 block {ms:.3f} ms ({tflops:.0f} TFLOP/s); stages (synchronized) ms {stages}")
    return {"ms": round(ms, 4), "tflops": round(tflops, 2), "linear_tflop": round(lin / 1e12, 4),
            "attention_tflop": round(att / 1e12, 4), "stage_ms": stages,
            "shape": {"tokens": KV_L, "hidden": 3072, "heads": KV_H, "cached_tokens": hist}}


def ar_chunk_flops(depth=40, prior=16, hidden=3072, heads=24, tokens=KV_L, d=KV_D, passes=5):
    """One AR chunk: `passes` passes of `depth` blocks, each block's linears plus
    attention over `prior` cached chunks and the current chunk."""
    lin, att = block_flops(hidden, heads, tokens, (prior + 1) * tokens, d)
    return passes * depth * (lin + att)


def bench_ar(args, torch, ops, dev, log):
    """Config 5: the 40-block AR step at the largest cache -- 4 denoising passes
    and 1 cache-write pass over 16 prior chunks (172 800 cached tokens per
    layer, FP8 codes written by the KV-write kernel)."""
    db = importlib.import_module("hy-nomas_amd.dit_block")
    depth, prior = 40, 16
    model = db.FP8ARModel(depth=depth, device=dev, seed=7)
    g = torch.Generator(device=dev).manual_seed(99)
    k = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
    for cache in model.caches:
        for c in range(prior):
            ops.kv_quantize_pair_(cache["k"], cache["v"], cache["k_scale"], cache["v_scale"],
                                  k, v, c * KV_L)
    del k, v
    model.cache_valid_len = prior * KV_L
    model.frames_done = prior * model.latent_shape[0]
    noise = torch.randn(1, KV_L, 3072, device=dev, generator=g).to(torch.bfloat16)
    vecs = [torch.randn(1, 3072, device=dev, generator=g).to(torch.bfloat16) for _ in range(5)]
    sigmas = torch.linspace(1.0, 0.0, 5).tolist()
    with torch.no_grad():
        model.forward_chunk(noise, vecs[0], update_cache=False)    # warm-up pass
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.generate_chunk(noise, vecs[:4], vecs[4], sigmas)
        torch.cuda.synchronize()
        sec = time.perf_counter() - t0
    flops = ar_chunk_flops(depth, prior)
    frames = model.latent_shape[0]
    log(f"config-5 AR chunk ({depth} blocks, {prior} prior chunks, 4+1 passes): {sec * 1e3:.0f} ms, "
        f"{frames / sec:.3f} latent frames/s, {flops / sec / 1e12:.0f} TFLOP/s")
    del model
    torch.cuda.empty_cache()
    return {"ms_per_chunk": round(sec * 1e3, 1), "latent_frames_per_s": round(frames / sec, 4),
            "tflops": round(flops / sec / 1e12, 1), "pflop_per_chunk": round(flops / 1e15, 3),
            "shape": {"blocks": depth, "prior_chunks": prior, "passes": "4 denoise + 1 cache write",
                      "tokens_per_chunk": KV_L, "cache_tokens_per_layer": prior * KV_L}}


def run_only(args, torch, ops, kvc, ca, dev, log):
    """One workload, for per-kernel counter passes (no JSON line)."""
    g = torch.Generator(device=dev).manual_seed(1234)
    if args.only == "linear":
        x = torch.randn(NS_M, NS_K, device=dev, generator=g).to(torch.bfloat16)
        w = (torch.randn(NS_N, NS_K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        bias = torch.zeros(NS_N, device=dev, dtype=torch.bfloat16)
        qw, sw = ops.quantize_rows_fp8(w)
        qx, sx = ops.quantize_rows_fp8(x)
        ms = time_loop(lambda: ops.gemm_fp8_rowcol(qx, qw, sx, sw, bias, 1), args.steps, args.warmup)
        log(f"north-star GEMM {ms:.3f} ms")
    elif args.only == "kv":
        # the config-2 layout of the main run: [1, H, L, D] data viewed as [1, L, H, D]
        k = torch.randn(1, KV_H, KV_L, KV_D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
        v = torch.randn(1, KV_H, KV_L, KV_D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
        cache = kvc.make_fp8_kv_block(1, KV_L, KV_H, KV_D, device=dev)
        ms = time_loop(lambda: ops.kv_quantize_pair_(cache["k"], cache["v"], cache["k_scale"],
                                                     cache["v_scale"], k, v, 0), args.steps, args.warmup)
        log(f"KV write {ms * 1e3:.1f} us")
    elif args.only == "attn":
        lk = ATT_CHUNKS * KV_L
        cache = kvc.make_fp8_kv_block(1, lk, KV_H, KV_D, device=dev)
        for c in range(ATT_CHUNKS):
            kc = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
            kvc.quantize_kv_pair_into(cache, kc, kc, c * KV_L)
        q = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
        ms = time_loop(lambda: ca.chunk_attention(q, cache, lk, q_pos0=lk - KV_L, chunk_len=KV_L),
                       args.steps, args.warmup)
        log(f"chunk attention {ms:.3f} ms")


def gemm_traffic_bytes():
    """HBM bytes per north-star GEMM launch from the committed counter summary
    (profiles/fp8_gemm_north_star_traffic.json), or None."""
    f = ROOT / "profiles" / "fp8_gemm_north_star_traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def cpu_baseline(seconds, log):
    """Oracle dequantize-then-matmul of a row sample of the north-star linear on
    the host's cores: per-token quant in C (1 thread), dequant + float64 BLAS matmul."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    from oracle import oracle as O

    cores = min(16, os.cpu_count() or 1)
    rng = np.random.default_rng(0)
    rows = 256
    x = rng.standard_normal((rows, NS_K)).astype(np.float32)
    w = (rng.standard_normal((NS_N, NS_K)) * 0.02).astype(np.float32)
    xb = O.f32_to_bf16_bits(x)
    qw, sw = O.quantize_rows_fp8(O.f32_to_bf16_bits(w))
    bias = rng.standard_normal(NS_N) * 0.01
    with threadpool_limits(limits=cores, user_api="blas"):
        blas = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
        n, t0 = 0, time.perf_counter()
        while True:
            qx, sx = O.quantize_rows_fp8(xb)
            O.linear_reference(qx, sx, qw, sw, bias, gelu=True)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 50:
                break
    tflops = gemm_flops(rows, NS_K, NS_N) * n / el / 1e12
    log(f"cpu baseline {tflops * 1e3:.2f} GFLOP/s over {n} x {rows} rows in {el:.1f} s")
    out = {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": int(blas[0]) if blas else cores,
           "kind": "port",
           "sample": f"{n} x {rows} token rows of the north-star linear ({rows}x{NS_K}x{NS_N}): "
                     f"oracle per-token e4m3 quant (C) + dequantize-then-matmul (numpy float64 BLAS) "
                     f"+ bias + GELU, {el:.1f} s"}
    out["kv_write"] = cpu_kv_write(O, seconds / 4, log)
    out["attention"] = cpu_attention(seconds / 2, cores, log)
    return out


def cpu_kv_write(O, seconds, log):
    """Config-2 recipe on the host (the reference CPU branch, int8_kv_cache.py:149-158, with
    448 and the e4m3 cast): the oracle's per-(token, head) quantizer in C, 1 thread, over
    a 1350-token x 24-head sample of K (1/8 of config 2's K), scaled to config 2's bytes."""
    import numpy as np
    rng = np.random.default_rng(1)
    L = KV_L // 8
    gain = rng.uniform(0.5, 4.0, KV_H).astype(np.float32)
    x = O.f32_to_bf16_bits((rng.standard_normal((1, L, KV_H, KV_D)) * gain[None, None, :, None]).astype(np.float32))
    n, t0 = 0, time.perf_counter()
    while True:
        O.kv_quantize(x)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 200:
            break
    rows = n * L * KV_H
    gbs = rows * (KV_D * 2 + KV_D + 4) / el / 1e9
    us_config2 = 2 * KV_L * KV_H * (el / rows) * 1e6
    log(f"cpu KV write {gbs:.2f} GB/s ({us_config2 / 1e3:.1f} ms for config 2's K and V)")
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "config2_ms_extrapolated": round(us_config2 / 1e3, 2),
            "sample": f"{n} x [1, {L}, {KV_H}, {KV_D}] bf16 rows through the oracle's KV quantizer (C), {el:.1f} s"}


def cpu_attention(seconds, cores, log):
    """Config-3 reference path on the host (nomas_cpt.py:771-781, attn_mode="torch"): decode
    the FP8 cache to bf16 with the reference's CPU branch (int8_kv_cache.py:202-204) and run
    torch's CPU scaled_dot_product_attention, for one head and a 64-query slice over all
    86 400 keys; TFLOP/s and the time extrapolated to config 3 (x 24 heads x 10800/64)."""
    import numpy as np
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(2)
    Lk, Lq = ATT_LK, 64
    codes = torch.from_numpy(rng.integers(0, 0x78, (2, Lk, KV_D), dtype=np.uint8)).view(torch.float8_e4m3fn)
    scales = torch.from_numpy(rng.uniform(1e-3, 1e-2, (2, Lk, 1)).astype(np.float32))
    q = torch.randn(1, 1, Lq, KV_D).to(torch.bfloat16)
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        n, t0 = 0, time.perf_counter()
        while True:
            kv = (codes.float() * scales).to(torch.bfloat16)   # the reference's CPU decode
            k, v = kv[0][None, None], kv[1][None, None]
            F.scaled_dot_product_attention(q, k, v, scale=KV_D ** -0.5)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 50:
                break
    finally:
        torch.set_num_threads(prev)
    flop = 4.0 * Lq * Lk * KV_D * n
    tflops = flop / el / 1e12
    ms3 = el / n * KV_H * (ATT_LQ / Lq) * 1e3
    log(f"cpu attention {tflops * 1e3:.1f} GFLOP/s ({ms3 / 1e3:.0f} s extrapolated to config 3)")
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": cores, "kind": "reference path (torch CPU)",
            "config3_s_extrapolated": round(ms3 / 1e3, 1),
            "sample": f"{n} x (decode 2 x {Lk} x {KV_D} FP8 codes + bf16 SDPA of {Lq} queries over "
                      f"{Lk} keys, one head), {el:.1f} s"}


if __name__ == "__main__":
    main()
