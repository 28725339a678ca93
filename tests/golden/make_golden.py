"""Write tests/golden/fp8_path_golden.npz: small input/expected-output vectors
for every function on the FP8 path.

The expected outputs come from torch CPU operations that restate the
reference's recipes step by step, not from oracle/:
  * per-token / per-channel / 128x128 FP8 quant: the torch ops of
    hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:35-41 (amax,
    clamp_min(1e-4), / 448, tensor division, .to(float8_e4m3fn)), with 1 x K
    blocks for the per-token form;
  * KV quantize-on-write, FP8 and INT8: hymm/models/dit/modules/int8_kv_cache.py:149-158
    (where(peak > 0, peak / Q, 1); FP8 uses Q = 448 and the e4m3 cast, INT8 the
    round-half-away / clamp steps);
  * linear: dequantize-then-matmul (int8_stored_bf16_linear.py:82-94 structure
    with e4m3 codes) in float64, bias, GELU-tanh;
  * chunk attention: softmax(Q K^T / sqrt(D)) V in float64 over K, V = code *
    scale with the chunk-granular visibility p // chunk <= r // chunk
    (nomas_cpt.py:368-376), fully masked rows zero (range_attention.py:212-239).
The oracle is checked against these vectors (tests/test_golden.py), and so are
the HIP kernels on the GPU, so the two are pinned independently of each other.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "fp8_path_golden.npz"
E4M3 = torch.float8_e4m3fn


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def codes(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def row_quant(xf: torch.Tensor, clamp: bool):
    amax = xf.abs().amax(dim=-1, keepdim=True)
    s = amax.clamp_min(1e-4) / 448.0 if clamp else torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    return (xf / s).to(E4M3), s


def main() -> None:
    g = torch.Generator().manual_seed(20261201)
    out = {}

    # ---- per-token activation quant: N(0,1) with x20 outliers, plus edge rows
    x = torch.randn(12, 384, generator=g)
    x[torch.rand(12, 384, generator=g) < 0.01] *= 20
    x[3] = 0.0                                   # zero row -> clamp floor
    x[4] = 0.0
    x[4, 17] = 448.0                             # amax 448 -> s = 1
    x[5] *= 1e-6                                 # below the 1e-4 floor
    x[6, :] = 3.0                                # constant row
    x[7, ::2] = -2.0 ** -12                      # subnormal codes after scaling
    xb = x.to(torch.bfloat16)
    q, s = row_quant(xb.float(), clamp=True)
    out.update(rows_x=bits(xb), rows_q=codes(q), rows_s=s[:, 0].numpy())
    q, s = row_quant(xb.float(), clamp=False)
    out.update(rows_q_zero_one=codes(q), rows_s_zero_one=s[:, 0].numpy())

    # ---- 128x128 blockwise quant, rows not a multiple of 128
    xw = (torch.randn(130, 256, generator=g) * 0.5).to(torch.bfloat16)
    m, k = xw.shape
    pad = torch.nn.functional.pad(xw.float(), (0, 0, 0, (-m) % 128))
    blocks = pad.reshape(-1, 128, k // 128, 128)
    sb = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-4) / 448.0
    qb = (blocks / sb[:, None, :, None]).to(E4M3).reshape(-1, k)[:m]
    out.update(block_x=bits(xw), block_q=codes(qb), block_s=sb.numpy())

    # ---- KV quantize-on-write, [B, L, H, D] = [1, 5, 3, 128], per-head gains
    gain = torch.tensor([0.5, 2.0, 4.0])
    kv = (torch.randn(1, 5, 3, 128, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
    kvf = kv.float().clone()
    kvf[0, 2, 1] = 0.0                          # zero row -> scale 1
    kv = kvf.to(torch.bfloat16)
    peak = kv.float().abs().amax(dim=-1, keepdim=True)
    s_fp8 = torch.where(peak > 0, peak / 448.0, torch.ones_like(peak))
    q_fp8 = (kv.float() / s_fp8).to(E4M3)
    s_i8 = torch.where(peak > 0, peak / 127.0, torch.ones_like(peak))
    scaled = kv.float() / s_i8
    q_i8 = torch.where(scaled >= 0, torch.floor(scaled + 0.5), torch.ceil(scaled - 0.5)).clamp(-127, 127).to(torch.int8)
    out.update(kv_x=bits(kv), kv_q_fp8=codes(q_fp8), kv_s_fp8=s_fp8.numpy(),
               kv_q_int8=q_i8.numpy(), kv_s_int8=s_i8.numpy())

    # ---- FP8 linear: x [9, 256] per-token, W [128, 256] per-channel, bias, GELU
    xl = torch.randn(9, 256, generator=g).to(torch.bfloat16)
    wl = (torch.randn(128, 256, generator=g) * 0.02).to(torch.bfloat16)
    bl = (torch.randn(128, generator=g) * 0.01).to(torch.bfloat16)
    qx, sx = row_quant(xl.float(), clamp=True)
    qw, sw = row_quant(wl.float(), clamp=True)
    y = (qx.double() * sx.double()) @ (qw.double() * sw.double()).T + bl.double()
    yg = 0.5 * y * (1 + torch.tanh(math.sqrt(2 / math.pi) * (y + 0.044715 * y ** 3)))
    out.update(lin_x=bits(xl), lin_w=bits(wl), lin_b=bits(bl), lin_qw=codes(qw), lin_sw=sw[:, 0].numpy(),
               lin_y=y.float().numpy(), lin_y_gelu=yg.float().numpy())

    # ---- chunk attention over an FP8 cache: 70 cached tokens, chunk 32,
    #      queries at positions 48..87 (two chunks: the triangle matters)
    H, D, kv_len, chunk, q0, Lq = 2, 128, 70, 32, 48, 40
    ka = (torch.randn(1, kv_len, H, D, generator=g) * 2).to(torch.bfloat16)
    va = torch.randn(1, kv_len, H, D, generator=g).to(torch.bfloat16)
    qa = torch.randn(1, Lq, H, D, generator=g).to(torch.bfloat16)
    kq, ks = row_quant(ka.float(), clamp=False)
    vq, vs = row_quant(va.float(), clamp=False)
    kh = kq.double() * ks.double()
    vh = vq.double() * vs.double()
    qpos = torch.arange(q0, q0 + Lq)
    kpos = torch.arange(kv_len)
    vis = (kpos[None, :] // chunk) <= (qpos[:, None] // chunk)
    o = torch.zeros(Lq, H, D, dtype=torch.float64)
    for h in range(H):
        logits = (qa[0, :, h].double() @ kh[0, :, h].T) / math.sqrt(D)
        logits = logits.masked_fill(~vis, float("-inf"))
        p = torch.softmax(logits, dim=-1)
        o[:, h] = p @ vh[0, :, h]
    out.update(att_q=bits(qa), att_kq=codes(kq), att_ks=ks.numpy(), att_vq=codes(vq), att_vs=vs.numpy(),
               att_o=o.float().numpy(), att_meta=np.array([H, D, kv_len, chunk, q0, Lq], np.int64))

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
