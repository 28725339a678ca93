"""The drop-in seams, exercised the way the reference's own code calls them:

* DiT linears: the compiled pre/post functions call F.linear(x, w, b) on
  ``linear_weight(module)`` (nomas_compile_prepost.py:45-47,80-87;
  nomas_cpt.py:1356-1370,1431-1441). With FP8StoredLinear modules that call,
  unchanged, runs the FP8 GEMM -- eagerly and under torch.compile, where the
  op stays one opaque node.
* convert_to_fp8, enable_fp8 and install_fp8 (reactor/hy_nomas_quantization.py:35-40)
  on stand-in modules."""
import types

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from conftest import assert_close_bf16, bf16_bits, pkg_module, u8

pytestmark = pytest.mark.gpu


class _Int8StandIn(nn.Module):
    """Only here so the reference's linear_weight has its INT8 branch to skip."""


def reference_linear_weight(module):
    """int8_stored_bf16_linear.py:97-100, unchanged in behaviour: the INT8
    class dequantizes, every other module gives its .weight."""
    if isinstance(module, _Int8StandIn):
        return module.dequant_weight()
    return module.weight


def reference_post_attention_img(img, img_attn, gate1, shift2, scale2, gate2, o_w, o_b, fc1_w, fc1_b,
                                 fc2_w, fc2_b):
    """The image half of nomas_compile_prepost.post_attention (:75-99), as written."""
    img = img + F.linear(img_attn, o_w, o_b) * gate1.unsqueeze(1)
    h = F.layer_norm(img, (img.shape[-1],), eps=1e-6) * (1 + scale2.unsqueeze(1)) + shift2.unsqueeze(1)
    h = F.linear(h, fc1_w, fc1_b)
    h = F.gelu(h, approximate="tanh")
    h = F.linear(h, fc2_w, fc2_b)
    return img + h * gate2.unsqueeze(1)


def _block(dev, hidden=256, mlp=4, seed=0):
    dl = pkg_module("dit_fp8_linear")
    g = torch.Generator(device=dev).manual_seed(seed)
    model = nn.ModuleDict({
        "proj": nn.Linear(hidden, hidden), "fc1": nn.Linear(hidden, mlp * hidden),
        "fc2": nn.Linear(mlp * hidden, hidden), "mod": nn.Linear(hidden, 6 * hidden)}).to(dev)
    with torch.no_grad():
        for m in model.values():
            m.weight.normal_(0, 0.02, generator=g)
            m.bias.normal_(0, 0.02, generator=g)
    model = model.to(torch.bfloat16)
    n = dl.convert_to_fp8(model, predicate=lambda name, m: name != "mod")
    assert n == 3
    assert isinstance(model["fc1"], dl.FP8StoredLinear) and isinstance(model["mod"], nn.Linear)
    return model


def test_unchanged_f_linear_call_runs_the_fp8_gemm(O, dev):
    dl = pkg_module("dit_fp8_linear")
    model = _block(dev)
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(2, 50, 1024, device=dev, generator=g).to(torch.bfloat16)
    fc2 = model["fc2"]
    w = reference_linear_weight(fc2)
    assert isinstance(w, dl.FP8Weight) and w.dtype == torch.bfloat16 and w.shape == (256, 1024)
    with torch.no_grad():
        y = F.linear(x, w, fc2.bias)
        assert torch.equal(y, fc2(x))                                   # the fused FP8 path
        assert not torch.equal(y, F.linear(x, fc2.dequant_weight(), fc2.bias))   # not the bf16 one
    # and against the oracle: per-token e4m3 x per-channel e4m3, fp32 accumulate, + bias
    qx, sx = O.quantize_rows_fp8(bf16_bits(x.reshape(-1, 1024)))
    ref = O.linear_reference(qx, sx, u8(fc2.weight_q), fc2.weight_scale.cpu().numpy(),
                             O.bf16_bits_to_f32(bf16_bits(fc2.bias)))
    assert_close_bf16(y.reshape(-1, 256).float().cpu().numpy(), ref, what="F.linear on FP8Weight")
    # any other use of the weight sees the reference's dequantized value
    assert torch.equal(w.float(), fc2.dequant_weight().float())
    assert torch.equal((w * 1).cpu(), fc2.dequant_weight().cpu())
    with pytest.raises(TypeError, match="BF16"):
        F.linear(x.float(), w, fc2.bias)


def _post_args(model, img, attn, parts):
    lw = reference_linear_weight
    return (img, attn, parts[2], parts[3], parts[4], parts[5],
            lw(model["proj"]), model["proj"].bias, lw(model["fc1"]), model["fc1"].bias,
            lw(model["fc2"]), model["fc2"].bias)


def test_reference_post_attention_unchanged_eager_and_compiled(dev):
    """The reference's post_attention body, fed linear_weight() of FP8 layers,
    equals the FP8 block path; torch.compile keeps the FP8 op as one opaque
    node (one graph, no breaks) and gives the same bits."""
    db = pkg_module("dit_block")
    dl = pkg_module("dit_fp8_linear")
    model = _block(dev, seed=2)
    g = torch.Generator(device=dev).manual_seed(3)
    img = torch.randn(1, 64, 256, device=dev, generator=g).to(torch.bfloat16)
    attn = torch.randn(1, 64, 256, device=dev, generator=g).to(torch.bfloat16)
    vec = torch.randn(1, 256, device=dev, generator=g).to(torch.bfloat16)
    parts = F.linear(F.silu(vec), model["mod"].weight, model["mod"].bias).chunk(6, dim=-1)
    with torch.no_grad():
        eager = reference_post_attention_img(*_post_args(model, img, attn, parts))
        # the FP8 block's own post-attention path (fused GEMM epilogues)
        x = img + dl.fp8_linear(model["proj"], attn) * parts[2].unsqueeze(1)
        h = db._modulate(F.layer_norm(x, (256,), eps=1e-6), parts[3], parts[4])
        h = dl.fp8_linear(model["fc1"], h, gelu=True)
        block = x + dl.fp8_linear(model["fc2"], h) * parts[5].unsqueeze(1)
    # the block fuses GELU into fc1's epilogue (its own exp2 form on the bf16
    # linear output); the reference applies F.gelu to the same bf16 values,
    # so the two differ by bf16 roundings only
    assert_close_bf16(eager.float().cpu().numpy(), block.float().cpu().numpy(), what="reference post vs block")
    torch._dynamo.reset()
    explain = torch._dynamo.explain(reference_post_attention_img)(*_post_args(model, img, attn, parts))
    assert explain.graph_count == 1 and explain.graph_break_count == 0
    compiled = torch.compile(reference_post_attention_img, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        out = compiled(*_post_args(model, img, attn, parts))
    assert torch.equal(out, eager)


def test_install_fp8_swaps_the_extension_seam(O, dev):
    """install_fp8 replaces the decoder module's load_extension, after which the
    reference's quantize-then-gemm call reaches the HIP blockwise GEMM."""
    quant = pkg_module("quantization")
    pf = pkg_module("pixelumm_fp8")
    calls = []
    stand_in = types.SimpleNamespace(load_extension=lambda: calls.append("cutlass") or None)
    quant.install_fp8(stand_in)
    ext = stand_in.load_extension()
    assert isinstance(ext, pf.HipFP8Extension) and not calls
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(200, 384, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(256, 384, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    qa, sa = pf.quantize_blockwise(x)       # cutlass_fp8._linear's two steps
    qb, sb = pf.quantize_blockwise(w)
    y = ext.gemm(qa, qb, sa, sb)
    ref = O.blockwise_gemm_reference(u8(qa), sa.cpu().numpy(), u8(qb), sb.cpu().numpy())
    got = y.float().cpu().numpy()
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 0.004
    with pytest.raises(RuntimeError, match="CUDA"):
        ext.gemm(qa.cpu(), qb, sa, sb)


def test_enable_fp8_on_a_stand_in_decoder(O, dev):
    pf = pkg_module("pixelumm_fp8")
    model = nn.Sequential(nn.Linear(256, 512, bias=False), nn.GELU(), nn.Linear(512, 256, bias=False))
    model = model.to(dev).to(torch.bfloat16).eval()
    with pytest.raises(ValueError, match="eval-mode"):
        pf.enable_fp8(model.train(), ["0", "2"])
    model.eval()
    biased = nn.Sequential(nn.Linear(256, 256)).to(dev).to(torch.bfloat16).eval()
    with pytest.raises(ValueError, match="bias-free"):
        pf.enable_fp8(biased, ["0"])
    assert pf.enable_fp8(model, ["0", "2"]) == 2
    assert isinstance(model[0], pf.FP8Linear) and isinstance(model[2], pf.FP8Linear)
    x = torch.randn(3, 7, 256, device=dev).to(torch.bfloat16)
    before = {(r["M"], r["K"], r["N"]): r["calls"] for r in pf.execution_stats()}
    with torch.no_grad():
        y = model(x)
    assert y.shape == (3, 7, 256) and torch.isfinite(y.float()).all()
    after = {(r["M"], r["K"], r["N"]): r["calls"] for r in pf.execution_stats()}
    assert after[(21, 256, 512)] == before.get((21, 256, 512), 0) + 1
    assert after[(21, 512, 256)] == before.get((21, 512, 256), 0) + 1
    with pytest.raises(RuntimeError, match="inference"):
        model[0](x)   # grad enabled
