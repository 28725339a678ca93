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

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-seconds S]
                       [--no-cpu-baseline] [--no-ar]
                       [--only all|linear|kv|attn|decode|blockwise|copy|ar]
``--only`` runs one workload (for per-kernel counter passes): ``attn`` config 3,
``decode`` 128 queries over the same 86 400-key cache, ``blockwise`` the decoder
layer's five blockwise-scaled FP8 GEMMs; ``copy`` is a plain 1 GiB device copy
used to calibrate the FETCH_SIZE / WRITE_SIZE counters; ``vendor`` times
hipBLASLt's FP8 GEMM (torch._scaled_mm, row-wise scales, no bias or
activation) beside this build's on the same operands.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import statistics
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
TEXT_TOKENS, TEXT_PAD = 256, 56              # text stream of the config-4 block's extra line


def gemm_flops(m, k, n):
    return 2.0 * m * k * n


def kv_write_bytes(h=KV_H, l=KV_L, d=KV_D):
    rows = 2 * h * l                     # K and V rows
    return rows * d * 2 + rows * d + rows * 4   # bf16 in, e4m3 out, fp32 scale out


def attn_flops(h, lq, lk, d):
    return 4.0 * h * lq * lk * d


def attn_unique_bytes(h, lq, lk, d):
    return h * lq * d * 2 * 2 + 2 * h * lk * d + 2 * h * lk * 4   # Q + O bf16, K/V codes, scales


def clock_settle(fn, seconds, torch):
    """Run fn back to back for a fixed wall-clock time (synchronizing every
    16 calls), so that the timed loops start at the GPU's steady clock."""
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(16):
            fn()
        calls += 16
        torch.cuda.synchronize()
    return {"seconds": round(time.perf_counter() - t0, 3), "calls": calls,
            "workload": "north-star FP8 linear, back to back, before any timed loop"}


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
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    # A GPU coming out of idle runs the first few hundred ms of dense FP8 work
    # at a moving clock (the north-star GEMM's calls drift from ~0.38 to
    # ~0.5 ms and back within the first ~30 calls); a fixed-length settle
    # phase of that same work precedes every timed workload, whatever
    # --warmup is, and is reported in the JSON line.
    ap.add_argument("--settle-seconds", type=float, default=3.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ar", action="store_true", help="skip the config-5 AR chunk (about 15 s)")
    ap.add_argument("--only", default="all",
                    choices=["all", "linear", "kv", "attn", "decode", "blockwise", "copy", "ar", "vendor",
                             "gemm_phases"])
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

    settle = clock_settle(lambda: ops.linear_fp8(x, qw, sw, bias, 1), args.settle_seconds, torch)
    log(f"clock settle: {settle['calls']} north-star linear calls in {settle['seconds']:.2f} s")
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

    # ---------------- decoder FP8 linears (blockwise 128x128 scales)
    dec_res = bench_decoder_linears(args, torch, ops, dev, g, log)

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

    # ---------------- the widened rows: fused kernels either side of the path, INT8-compat KV
    wide_res = bench_widened(args, torch, kvc, ca, dev, g, lib, L, stream_ptr, log)

    # ---------------- config 4: one FP8 DiT block over 7 cached chunks + the current one
    blk_res = bench_block(args, torch, cache, dev, g, log)
    del cache, q, qd

    # ---------------- config 5: 40-block AR chunk at the largest cache
    ar_res = bench_ar(args, torch, ops, dev, log) if not args.no_ar else None

    # ---------------- CPU baseline: the reference's own torch CPU paths
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(log)

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
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over this GEMM "
                              "(profiles/hbm_traffic.json: workloads.linear_gemm), scaled by the same "
                              "counters over a 1 GiB copy; not measured inside this run",
        },
        # every hot kernel of the step against its own roofline (the GEMM
        # repeated from `roofline`); attention entries time the whole call
        # (its launches and the split merge)
        "rooflines": [
            roofline_entry("gemm_rowcol_oe_kernel: north-star FP8 GEMM + bias + GELU", "mfma", f_ns,
                           "flop", ms_gemm, FP8_PEAK_TFLOPS, "TFLOP/s", "linear_gemm"),
            roofline_entry("kv_quantize_kernel: config-2 K and V write", "hbm", kv_write_bytes(),
                           "byte", ms_kv, HBM_PEAK_GBS, "GB/s", "kv_write"),
            roofline_entry("attn_fp8kv_kernel: config-3 chunk attention (bf16 MFMA over e4m3 K/V)",
                           "mfma", attn_flops(KV_H, KV_L, lk, KV_D), "flop", ms_att, BF16_PEAK_TFLOPS,
                           "TFLOP/s", "attn_config3"),
            roofline_entry("attn_fp8kv_kernel + attn_combine_kernel: decode-style attention, "
                           "Lq 128 over 86 400 cached keys", "hbm", attn_unique_bytes(KV_H, 128, lk, KV_D),
                           "byte", ms_dec, HBM_PEAK_GBS, "GB/s", "attn_decode"),
        ],
        "clock_settle": settle,
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
        "decoder_blockwise": dec_res,
        "widened": wide_res,
        "dit_block": blk_res,
        "ar_chunk": ar_res,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))


def bench_widened(args, torch, kvc, ca, dev, g, lib, L, stream_ptr, log):
    """The kernels beside the hot path, each at the block's shapes:
    * LayerNorm + adaLN modulate + per-token e4m3 quant of the block input,
      10800 x 3072 (the input of QKV and of fc1);
    * QK RMSNorm + RoPE in place on the QKV output with the K/V cache write in
      the same kernel (the AR write pass), 10800 tokens x 24 heads;
    * the reference's own INT8 KV format: the config-2 write and the config-3
      and decode-style attention over an INT8 cache.
    Short kernels go through the C ABI with preallocated outputs. Algorithmic
    bytes: LN + quant 2 C + C + 4 per row; QK + write reads q, k, v and the
    fp32 cos/sin tables, writes q, k, the K/V codes and their scales."""
    bf, f8 = torch.bfloat16, torch.float8_e4m3fn
    res = {}
    x = torch.randn(1, NS_M, NS_K, device=dev, generator=g).to(bf)
    shift = (torch.randn(1, NS_K, device=dev, generator=g) * 0.1).to(bf)
    scale = (torch.randn(1, NS_K, device=dev, generator=g) * 0.1).to(bf)
    qx = torch.empty(NS_M, NS_K, dtype=f8, device=dev)
    sx = torch.empty(NS_M, dtype=torch.float32, device=dev)
    ln_args = (x.data_ptr(), NS_M, NS_K, NS_M, shift.data_ptr(), scale.data_ptr(), NS_K, 1e-6, 1e-4,
               qx.data_ptr(), sx.data_ptr(), stream_ptr)
    L.check(lib.hn_ln_mod_quantize_fp8(*ln_args), "hn_ln_mod_quantize_fp8")
    ms = time_loop(lambda: lib.hn_ln_mod_quantize_fp8(*ln_args), args.steps, args.warmup)
    nbytes = NS_M * NS_K * 3 + NS_M * 4
    res["ln_mod_quant"] = {"us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "shape": [NS_M, NS_K]}
    log(f"LayerNorm + modulate + quant {ms * 1e3:.1f} us ({nbytes / (ms * 1e-3) / 1e9:.0f} GB/s)")
    del x, qx

    H, D = KV_H, KV_D
    qkv = torch.randn(1, KV_L, 3, H, D, device=dev, generator=g).to(bf)
    q, k, v = qkv.unbind(2)
    qw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(bf)
    kw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(bf)
    ang = torch.rand(KV_L, D, device=dev, generator=g) * 6.283
    cos, sin = torch.cos(ang), torch.sin(ang)
    cache = kvc.make_fp8_kv_block(1, KV_L, H, D, device=dev)
    qk_args = (L.HN_KV_FP8, q.data_ptr(), k.data_ptr(), v.data_ptr(), L.strides(q), 1, KV_L, H, D,
               qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.stride(0), 1e-6,
               cache["k"].data_ptr(), cache["v"].data_ptr(), L.strides(cache["k"]),
               cache["k_scale"].data_ptr(), cache["v_scale"].data_ptr(), L.strides(cache["k_scale"]),
               KV_L, 0, None, stream_ptr)
    L.check(lib.hn_qk_norm_rope_kv(*qk_args), "hn_qk_norm_rope_kv")
    ms = time_loop(lambda: lib.hn_qk_norm_rope_kv(*qk_args), args.steps, args.warmup)
    rows = KV_L * H
    nbytes = rows * D * 2 * 3 + 2 * KV_L * D * 4 + rows * D * 2 * 2 + rows * D * 2 + rows * 4 * 2
    res["qk_norm_rope_kv_write"] = {"us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                    "shape": [1, KV_L, H, D]}
    log(f"QK RMSNorm + RoPE + KV write {ms * 1e3:.1f} us ({nbytes / (ms * 1e-3) / 1e9:.0f} GB/s)")
    del qkv, q, k, v, cache

    # INT8-compat KV (the reference's kv_cache_quantization=int8 format)
    lk = ATT_CHUNKS * KV_L
    cache = kvc.make_int8_kv_block(1, lk, H, D, device=dev)
    gain = torch.empty(H, device=dev).uniform_(0.5, 4.0, generator=g)
    kb = (torch.randn(1, H, KV_L, D, device=dev, generator=g) * gain[None, :, None, None]).to(bf).transpose(1, 2)
    vb = (torch.randn(1, H, KV_L, D, device=dev, generator=g) * gain[None, :, None, None]).to(bf).transpose(1, 2)
    kv_args = (L.HN_KV_INT8, kb.data_ptr(), vb.data_ptr(), L.strides(kb), 1, KV_L, H, D,
               cache["k"].data_ptr(), cache["v"].data_ptr(), L.strides(cache["k"]),
               cache["k_scale"].data_ptr(), cache["v_scale"].data_ptr(), L.strides(cache["k_scale"]),
               lk, (ATT_CHUNKS - 1) * KV_L, None, stream_ptr)
    L.check(lib.hn_kv_quantize_pair(*kv_args), "hn_kv_quantize_pair")
    ms_kv = time_loop(lambda: lib.hn_kv_quantize_pair(*kv_args), args.steps, args.warmup)
    for c in range(ATT_CHUNKS):
        gain = torch.empty(H, device=dev).uniform_(0.5, 4.0, generator=g)
        kc = (torch.randn(1, KV_L, H, D, device=dev, generator=g) * gain[None, None, :, None]).to(bf)
        vc = (torch.randn(1, KV_L, H, D, device=dev, generator=g) * gain[None, None, :, None]).to(bf)
        kvc.quantize_kv_pair_into(cache, kc, vc, c * KV_L)
    del kc, vc, kb, vb
    qa = torch.randn(1, KV_L, H, D, device=dev, generator=g).to(bf)
    ms_att = time_loop(lambda: ca.chunk_attention(qa, cache, lk, q_pos0=lk - KV_L, chunk_len=KV_L),
                       max(2, args.steps // 4), max(1, args.warmup // 2))
    qd = qa[:, :128].contiguous()
    ms_dec = time_loop(lambda: ca.chunk_attention(qd, cache, lk), args.steps, args.warmup)
    kv_gbs = kv_write_bytes() / (ms_kv * 1e-3) / 1e9
    att_tflops = attn_flops(H, KV_L, lk, D) / (ms_att * 1e-3) / 1e12
    dec_gbs = attn_unique_bytes(H, 128, lk, D) / (ms_dec * 1e-3) / 1e9
    res["int8_kv"] = {"write_us": round(ms_kv * 1e3, 2), "write_gbs": round(kv_gbs, 1),
                      "attention_ms": round(ms_att, 4), "attention_tflops": round(att_tflops, 2),
                      "decode_lq128_us": round(ms_dec * 1e3, 2), "decode_lq128_gbs": round(dec_gbs, 1)}
    log(f"INT8 KV: write {ms_kv * 1e3:.1f} us ({kv_gbs:.0f} GB/s); chunk attention {ms_att:.3f} ms "
        f"({att_tflops:.0f} TFLOP/s); decode-style {ms_dec * 1e3:.1f} us ({dec_gbs:.0f} GB/s)")
    return res


# The PixelUMM decoder layer's FP8 linears (pixelumm_decoder/model.py:43-53,
# 203-206,263-265; cutlass_fp8.py:106-121 converts q/o/gate/up/down): hidden
# 4096, FFN 12288, over one 10800-token window (3 latent frames of 45 x 80).
DEC_M = 10800
DEC_LINEARS = (("q_proj", 4096, 4096), ("o_proj", 4096, 4096), ("gate_proj", 4096, 12288),
               ("up_proj", 4096, 12288), ("down_proj", 12288, 4096))


def bench_decoder_linears(args, torch, ops, dev, g, log):
    """Blockwise-scaled FP8 GEMMs (the reference's gemm(a, b, sa, sb)) at the
    decoder layer's five FP8 linear shapes, operands quantized once outside
    the timed loop."""
    pf = importlib.import_module("hy-nomas_amd.pixelumm_fp8")
    out, total_ms, total_flop = {}, 0.0, 0.0
    for name, k, n in DEC_LINEARS:
        a = torch.randn(DEC_M, k, device=dev, generator=g).to(torch.bfloat16)
        b = (torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        qa, sa = pf.quantize_blockwise(a)
        qb, sb = pf.quantize_blockwise(b)
        del a, b
        ms = time_loop(lambda: ops.gemm_fp8_blockwise(qa, qb, sa, sb), args.steps, args.warmup)
        flop = gemm_flops(DEC_M, k, n)
        tf = flop / (ms * 1e-3) / 1e12
        out[name] = {"mkn": [DEC_M, k, n], "us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                     "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)}
        total_ms += ms
        total_flop += flop
    tf = total_flop / (total_ms * 1e-3) / 1e12
    log(f"decoder FP8 linears (blockwise, M={DEC_M}): {total_ms:.3f} ms per layer, {tf:.0f} TFLOP/s; "
        + ", ".join(f"{k} {v['us']:.0f} us" for k, v in out.items()))
    out["layer"] = {"ms": round(total_ms, 4), "tflops": round(tf, 1), "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)}
    return out


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
    res = {"ms": round(ms, 4), "tflops": round(tflops, 2), "linear_tflop": round(lin / 1e12, 4),
           "attention_tflop": round(att / 1e12, 4), "stage_ms": stages,
           "shape": {"tokens": KV_L, "hidden": 3072, "heads": KV_H, "cached_tokens": hist}}
    # The same block with the double-stream block's text stream (BASELINE's
    # config 4 names none): TEXT_TOKENS text tokens, the last TEXT_PAD of them
    # padding, a segment's first chunk (cache_txt), denoise pass: queries
    # [img | txt] over [7 cached chunks | img | txt] with the text mask.
    del blk
    tblk = db.FP8DiTBlock(3072, KV_H, device=dev, generator=g, text=True)
    txt = torch.randn(1, TEXT_TOKENS, 3072, device=dev, generator=g).to(torch.bfloat16)
    vec_txt = torch.randn(1, 3072, device=dev, generator=g).to(torch.bfloat16)
    tmask = torch.ones(1, TEXT_TOKENS, dtype=torch.bool, device=dev)
    tmask[0, TEXT_TOKENS - TEXT_PAD:] = False
    cmask = torch.ones(1, cache["k"].shape[1], dtype=torch.bool, device=dev)
    tfn = lambda: tblk(img, vec, cos, sin, cache, hist, False, txt=txt, vec_txt=vec_txt,
                       text_mask=tmask, cache_mask=cmask, cache_txt=True)
    with torch.no_grad():
        tms = time_loop(tfn, max(2, args.steps // 4), max(1, args.warmup // 2))
    tl, ta = block_flops(tokens=KV_L + TEXT_TOKENS, keys=hist + KV_L + TEXT_TOKENS)
    log(f"config-4 block with {TEXT_TOKENS} text tokens {tms:.3f} ms "
        f"({(tl + ta) / (tms * 1e-3) / 1e12:.0f} TFLOP/s)")
    res["with_text"] = {"ms": round(tms, 4), "text_tokens": TEXT_TOKENS, "text_padding": TEXT_PAD,
                        "tflops": round((tl + ta) / (tms * 1e-3) / 1e12, 2)}
    return res


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
    elif args.only == "blockwise":
        bench_decoder_linears(args, torch, ops, dev, g, log)
    elif args.only == "vendor":
        # hipBLASLt (through torch._scaled_mm: out = (a sa) (b sb)^T in bf16)
        # against hn_gemm_fp8_rowcol without bias or activation, same operands.
        a = torch.randn(NS_M, NS_K, device=dev, generator=g).to(torch.bfloat16)
        qa, sa = ops.quantize_rows_fp8(a)
        settle = clock_settle(lambda: ops.gemm_fp8_rowcol(qa, qa[:NS_K], sa, sa[:NS_K]), args.settle_seconds, torch)
        log(f"clock settle: {settle['calls']} GEMM calls in {settle['seconds']:.2f} s")
        for (m, k, n) in ((NS_M, NS_K, NS_N), (C1_M, C1_K, C1_N), (NS_M, NS_N, NS_K), (8192, 8192, 8192)):
            qa, sa = ops.quantize_rows_fp8(torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16))
            qb, sb = ops.quantize_rows_fp8((torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16))
            ours = time_loop(lambda: ops.gemm_fp8_rowcol(qa, qb, sa, sb), args.steps, args.warmup)
            sa2, sb2 = sa.view(m, 1), sb.view(1, n)
            theirs = time_loop(lambda: torch._scaled_mm(qa, qb.t(), scale_a=sa2, scale_b=sb2,
                                                        out_dtype=torch.bfloat16), args.steps, args.warmup)
            diff = (ops.gemm_fp8_rowcol(qa, qb, sa, sb).float()
                    - torch._scaled_mm(qa, qb.t(), scale_a=sa2, scale_b=sb2, out_dtype=torch.bfloat16).float())
            tf = gemm_flops(m, k, n) / 1e9
            log(f"{m}x{k}x{n}: hn_gemm_fp8_rowcol {ours * 1e3:.1f} us ({tf / ours:.0f} TFLOP/s), "
                f"hipBLASLt {theirs * 1e3:.1f} us ({tf / theirs:.0f} TFLOP/s), max |diff| {diff.abs().max().item():.3g}")
    elif args.only == "gemm_phases":
        bench_gemm_phases(args, torch, ops, dev, g, log)
    elif args.only in ("attn", "decode"):
        lk = ATT_CHUNKS * KV_L
        cache = kvc.make_fp8_kv_block(1, lk, KV_H, KV_D, device=dev)
        for c in range(ATT_CHUNKS):
            kc = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
            kvc.quantize_kv_pair_into(cache, kc, kc, c * KV_L)
        if args.only == "attn":
            q = torch.randn(1, KV_L, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
            ms = time_loop(lambda: ca.chunk_attention(q, cache, lk, q_pos0=lk - KV_L, chunk_len=KV_L),
                           args.steps, args.warmup)
            log(f"chunk attention {ms:.3f} ms")
        else:
            q = torch.randn(1, 128, KV_H, KV_D, device=dev, generator=g).to(torch.bfloat16)
            ms = time_loop(lambda: ca.chunk_attention(q, cache, lk), args.steps, args.warmup)
            log(f"decode-style attention (Lq=128) {ms * 1e3:.1f} us")


STAMP_SHAPE = (16, 12, 8)   # workgroups x tiles x phases recorded by the stamps library
STAMP_PHASES = ("steps 0-4, carrying the previous tile's epilogue", "steps 5 .. KT-1", "end-of-loop barrier",
                "next tile's step-1 loads", "direct epilogue passes", "conversion of the carried rows",
                "wait for the next tile's step 0 + barrier")


def bench_gemm_phases(args, torch, ops, dev, g, log):
    """Where a persistent-GEMM tile's cycles go: the measurement library
    libhynomas_fp8_stamps.so (the same kernel, compiled with
    HN_GEMM_PHASE_STAMPS) records the shader clock (s_memtime) at each phase
    boundary of workgroups 0-15's first 12 tiles. Per shape: the time per call,
    then the median cycles of each phase over those workgroups' whole tiles.
    HN_GEMM_WG_PER_XCD (environment) caps the launch's workgroups per XCD."""
    import ctypes
    import numpy as np
    lib = ctypes.CDLL(str(ROOT / "hy-nomas_amd" / "libhynomas_fp8_stamps.so"))
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    lib.hn_gemm_fp8_rowcol.argtypes = [P, P, P, P, P, P, I64, I64, I64, I64, ctypes.c_int, P]
    lib.hn_gemm_phase_stamps.argtypes = [P, I64, ctypes.c_int]
    nbytes = int(np.prod(STAMP_SHAPE)) * 8
    cap = os.environ.get("HN_GEMM_WG_PER_XCD", "all")
    for (m, n, k, act) in ((NS_M, NS_N, NS_K, 1), (10752, NS_N, NS_K, 0), (8192, 12288, 12288, 0)):
        x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        w = (torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        qx, sx = ops.quantize_rows_fp8(x)
        qw, sw = ops.quantize_rows_fp8(w)
        del x, w
        bias = torch.zeros(n, device=dev, dtype=torch.bfloat16)
        out = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        stream = torch.cuda.current_stream().cuda_stream

        def call():
            rc = lib.hn_gemm_fp8_rowcol(qx.data_ptr(), qw.data_ptr(), sx.data_ptr(), sw.data_ptr(),
                                        bias.data_ptr(), out.data_ptr(), m, n, k, n, act, stream)
            if rc:
                raise RuntimeError(f"stamps GEMM failed ({rc})")
        ms = time_loop(call, args.steps, args.warmup)
        if lib.hn_gemm_phase_stamps(None, nbytes, 1):
            raise RuntimeError("clearing the phase stamps failed")
        call()
        torch.cuda.synchronize()
        st = np.zeros(STAMP_SHAPE, dtype=np.uint64)
        if lib.hn_gemm_phase_stamps(st.ctypes.data, nbytes, 0):
            raise RuntimeError("reading the phase stamps failed")
        st = st.astype(np.int64)
        whole = (st[:, :, 0] > 0) & (st[:, :, 1] > 0) & (st[:, :, 7] > 0)   # whole tiles stamp phase 1
        d = np.diff(st, axis=2)[whole]                                      # [tiles, 7] cycles per phase
        med = np.median(d, axis=0)
        tot = float(np.median(d.sum(axis=1)))
        log(f"{m}x{n}x{k} act {act} (workgroups per XCD: {cap}): {ms * 1e3:.1f} us per call; "
            f"{len(d)} whole tiles, median {tot:.0f} cycles per tile")
        for name, c in zip(STAMP_PHASES, med):
            log(f"    {name:44s} {c:8.0f} cycles  {100 * c / tot:5.1f} %")
        log(f"    per K step: steps 5 .. KT-1 {med[1] / (k // 128 - 5):.0f} cycles, steps 0-4 {med[0] / 5:.0f}")


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.json"


def counter_traffic(workload):
    """HBM bytes per call of ``workload`` from the committed counter summary
    (profiles/hbm_traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE passes,
    scaled by the same counters over a plain copy), or None. Not measured in
    this run: the counters need a rocprofv3 pass of their own."""
    if not TRAFFIC_FILE.exists():
        return None
    try:
        entry = json.loads(TRAFFIC_FILE.read_text())["workloads"].get(workload)
    except (ValueError, OSError, KeyError):
        return None
    return None if entry is None else entry.get("hbm_bytes_per_call")


def gemm_traffic_bytes():
    """HBM bytes per north-star GEMM launch (profiles/hbm_traffic.json), or None."""
    return counter_traffic("linear_gemm")


def roofline_entry(name, bound, work, unit_work, ms, peak, unit, traffic_key):
    """One kernel's position against its roofline: ``work`` algorithmic flop
    or bytes per call over the measured ms per call, against ``peak``."""
    rate = work / (ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
    return {"kernel": name, "bound": bound, "work_per_call": work, "work_unit": unit_work,
            "ms_per_call": round(ms, 5), "achieved": round(rate, 2), "peak": peak, "unit": unit,
            "frac": round(rate / peak, 4), "traffic": counter_traffic(traffic_key),
            "traffic_source": f"profiles/hbm_traffic.json: workloads.{traffic_key}"}


def _median_seconds(fn, reps=5, warmup=2):
    """Median wall time of ``reps`` calls of fn after ``warmup`` untimed ones."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def _cpu_threads(torch, log):
    """Thread count for the CPU legs: the fastest of os.cpu_count(), the
    process's CPU affinity and OMP_NUM_THREADS (the GPU box grants each GPU a
    share of the host's CPUs; threads beyond that share only contend), picked
    on a short bf16 matmul probe."""
    cands = {os.cpu_count() or 1, len(os.sched_getaffinity(0))}
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cands.add(int(os.environ["OMP_NUM_THREADS"]))
    a = torch.randn(128, NS_K).to(torch.bfloat16)
    b = torch.randn(4096, NS_K).to(torch.bfloat16)
    probe = {}
    for n in sorted(cands):
        torch.set_num_threads(n)
        probe[n] = _median_seconds(lambda: torch.nn.functional.linear(a, b), reps=3, warmup=1)
    best = min(probe, key=probe.get)
    log(f"cpu threads probe (s per 128x3072x4096 bf16 matmul): {probe} -> {best}")
    return best, {str(k): round(v, 5) for k, v in probe.items()}


def cpu_baseline(log):
    """The reference's own CPU paths for the three kernels, in torch on the
    host's cores (2 warm-up calls, median of 5 timed ones per leg); each leg
    times a bounded sample and states how it scales to the full workload."""
    import torch
    prev = torch.get_num_threads()
    cores, probe = _cpu_threads(torch, log)
    torch.set_num_threads(cores)
    try:
        out = cpu_linear(torch, cores, log)
        out["threads_probe_s"] = probe
        out["kv_write"] = cpu_kv_write(torch, cores, log)
        out["attention"] = cpu_attention(torch, cores, log)
    finally:
        torch.set_num_threads(prev)
    return out


def cpu_linear(torch, cores, log):
    """North-star linear through the reference's module path on the CPU
    (int8_stored_bf16_linear.py:82-94 with e4m3 codes and per-channel scales):
    dequant_weight() = codes.float() * scale -> bf16, F.linear(x, w, bias) in
    bf16, then GELU-tanh (nomas_compile_prepost.py:83-84). The weight decode is
    timed whole (it does not depend on M); the bf16 GEMM on a row sample sized
    to about a second per call, scaled to M = 10800."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(0)
    codes = (torch.randn(NS_N, NS_K, generator=g) * 0.02 / 1e-4).clamp(-448, 448).to(torch.float8_e4m3fn)
    scale = torch.full((NS_N, 1), 1e-4)
    bias = (torch.randn(NS_N, generator=g) * 0.01).to(torch.bfloat16)
    w = (codes.float() * scale).to(torch.bfloat16)

    def dequant():
        return (codes.float() * scale).to(torch.bfloat16)

    def gemm(x):
        return F.gelu(F.linear(x, w, bias), approximate="tanh")

    x64 = torch.randn(64, NS_K, generator=g).to(torch.bfloat16)
    t64 = _median_seconds(lambda: gemm(x64), reps=1, warmup=1)
    rows = int(max(64, 64 * 1.0 / max(t64, 1e-6))) // 64 * 64
    rows = NS_M if rows >= NS_M else rows
    x = torch.randn(rows, NS_K, generator=g).to(torch.bfloat16)
    t_dq = _median_seconds(dequant)
    t_rows = _median_seconds(lambda: gemm(x))
    t_full = t_dq + t_rows * NS_M / rows
    tflops = gemm_flops(NS_M, NS_K, NS_N) / t_full / 1e12
    log(f"cpu linear (torch reference path): dequant {t_dq * 1e3:.1f} ms + {rows}-row bf16 GEMM+GELU "
        f"{t_rows * 1e3:.1f} ms -> {t_full:.2f} s at M={NS_M}, {tflops * 1e3:.2f} GFLOP/s")
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": cores,
            "kind": "reference path (torch CPU)",
            "north_star_s_extrapolated": round(t_full, 3),
            "sample": f"dequant_weight of the [{NS_N}, {NS_K}] e4m3 weight (whole, {t_dq * 1e3:.1f} ms) + "
                      f"bf16 F.linear + bias + GELU-tanh on {rows} of {NS_M} token rows ({t_rows * 1e3:.1f} ms), "
                      f"median of 5 after 2 warm-ups each; full M = dequant + GEMM x {NS_M}/{rows}"}


def cpu_kv_write(torch, cores, log):
    """Config 2 through the reference's CPU write branch (int8_kv_cache.py:149-158)
    with the FP8 constants: per (token, head) peak over D, s = peak / 448
    (1 where the peak is 0), codes = e4m3(x / s); K then V, at full size."""
    g = torch.Generator().manual_seed(1)
    gain = torch.empty(KV_H).uniform_(0.5, 4.0, generator=g)
    k = (torch.randn(1, KV_L, KV_H, KV_D, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
    v = (torch.randn(1, KV_L, KV_H, KV_D, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
    q = torch.empty(2, 1, KV_L, KV_H, KV_D, dtype=torch.float8_e4m3fn)
    sc = torch.empty(2, 1, KV_L, KV_H, 1)

    def write():
        for i, values in enumerate((k, v)):
            src = values.float()
            peak = src.abs().amax(dim=-1, keepdim=True)
            s = torch.where(peak > 0, peak / 448.0, torch.ones_like(peak))
            q[i].copy_((src / s).to(torch.float8_e4m3fn))
            sc[i].copy_(s)

    t = _median_seconds(write)
    gbs = kv_write_bytes() / t / 1e9
    log(f"cpu KV write (torch reference branch): {t * 1e3:.1f} ms for config 2, {gbs:.2f} GB/s")
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": cores, "kind": "reference path (torch CPU)",
            "config2_ms": round(t * 1e3, 2),
            "sample": f"config 2 whole: K and V [1, {KV_L}, {KV_H}, {KV_D}] bf16 -> e4m3 codes + fp32 scales, "
                      "median of 5 after 2 warm-ups"}


def cpu_attention(torch, cores, log):
    """Config-3 reference path on the host (nomas_cpt.py:771-781, attn_mode
    "torch"): decode the FP8 cache to bf16 with the reference's CPU branch
    (int8_kv_cache.py:202-204), then torch's CPU scaled_dot_product_attention.
    Sample: the decode of one head's K and V (86 400 keys) and the SDPA of
    one head's 64-query slice over all keys; config 3 = 24 heads' decode plus
    24 x 10800/64 such slices."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(2)
    Lk, Lq = ATT_LK, 64
    codes = torch.randint(0, 0x78, (2, 1, Lk, 1, KV_D), dtype=torch.uint8, generator=g).view(torch.float8_e4m3fn)
    scales = torch.empty(2, 1, Lk, 1, 1).uniform_(1e-3, 1e-2, generator=g)
    q = torch.randn(1, 1, Lq, KV_D, generator=g).to(torch.bfloat16)
    kv = (codes.float() * scales).to(torch.bfloat16)
    k, v = kv[0].transpose(1, 2), kv[1].transpose(1, 2)   # [1, 1, Lk, D]

    def decode():
        return (codes.float() * scales).to(torch.bfloat16)

    t_dec = _median_seconds(decode)
    t_sdpa = _median_seconds(lambda: F.scaled_dot_product_attention(q, k, v, scale=KV_D ** -0.5))
    t_full = KV_H * t_dec + KV_H * (ATT_LQ / Lq) * t_sdpa
    tflops = attn_flops(KV_H, ATT_LQ, Lk, KV_D) / t_full / 1e12
    log(f"cpu attention (torch reference path): decode {t_dec * 1e3:.1f} ms/head, SDPA {t_sdpa * 1e3:.1f} ms "
        f"per 64 queries -> {t_full:.0f} s for config 3, {tflops * 1e3:.2f} GFLOP/s")
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": cores, "kind": "reference path (torch CPU)",
            "config3_s_extrapolated": round(t_full, 1),
            "sample": f"decode of one head's K and V ({Lk} keys, {t_dec * 1e3:.1f} ms) + bf16 SDPA of {Lq} "
                      f"queries over {Lk} keys ({t_sdpa * 1e3:.1f} ms), median of 5 after 2 warm-ups each; "
                      f"config 3 = {KV_H} x decode + {KV_H} x {ATT_LQ}/{Lq} x SDPA"}


if __name__ == "__main__":
    main()
