"""The FP8 KV storage binding on a stand-in of the reference's AR pipeline
(tests/standin_pipeline.py): selection of ``kv_cache_quantization: fp8``
(causal_ar.py:357-361), allocation down the quantized branch
(causal_ar.py:589-594), capacity growth (:632-690) and the end-of-generation
audit the pipeline assembles (:3365-3374) from cache_storage_audit
(kv_cache_storage.py:77-105). CPU only: the write through the attention seam
is covered by tests/test_gpu_attention.py::test_pipeline_fp8_storage_write_and_audit."""
import pytest
import torch

from conftest import pkg_module
from standin_pipeline import args_for, make_reference

AUDIT_KEYS = {"storage_format", "gpu_storage_bytes", "storage_dtypes", "codec_stats",
              "peak_working_bytes", "transfer_bytes_scope"}


def _fp8_bytes(B, cap, H, D):
    return 2 * B * cap * H * D + 2 * B * cap * H * 4


def test_reference_refuses_fp8_until_installed():
    storage, int8_kv, Pipeline = make_reference()
    with pytest.raises(ValueError, match="none, int8, or qvg"):
        Pipeline(args_for("fp8"))
    st = pkg_module("kv_cache_storage")
    hook = st.install_fp8_kv_storage(storage, pipeline_cls=Pipeline, int8_kv_module=int8_kv)
    try:
        pipe = Pipeline(args_for("fp8"))
        assert pipe.kv_storage_format == "fp8" and not pipe.int8_kv_storage
        with pytest.raises(ValueError, match="none, int8, or qvg"):
            Pipeline(args_for("int4"))            # other modes: the module's own rule
    finally:
        hook.uninstall()
    with pytest.raises(ValueError):
        Pipeline(args_for("fp8"))


def test_pipeline_allocates_fp8_blocks_and_audits_them():
    storage, int8_kv, Pipeline = make_reference()
    st = pkg_module("kv_cache_storage")
    make0, init0 = int8_kv.make_int8_kv_block, Pipeline.__dict__["_initialize_kv_cache"]
    hook = st.install_fp8_kv_storage(storage, pipeline_cls=Pipeline, int8_kv_module=int8_kv)
    try:
        pipe = Pipeline(args_for("fp8"), hidden_size=256, heads_num=2, num_double_blocks=3)
        B, cap, H, D = 2, 40, 2, 128
        pipe._initialize_kv_cache(B, cap, torch.bfloat16, "cpu")
        assert hook.stats["fp8_allocations"] == 1
        # the INT8 module and the pipeline flag are as they were
        assert int8_kv.make_int8_kv_block is make0 and pipe.int8_kv_storage is False
        assert pipe.log == ["format=int8"]          # the pipeline's own log names its branch
        assert len(pipe.kv_cache) == 3 and len(pipe.cache_mask_list) == 3
        for cache in pipe.kv_cache:
            assert cache["k"].dtype == cache["v"].dtype == torch.float8_e4m3fn
            assert cache["k"].shape == (B, cap, H, D)
            assert cache["k_scale"].shape == cache["v_scale"].shape == (B, cap, H, 1)
            assert cache["k_scale"].dtype == torch.float32
            assert storage.cache_format(cache) == "fp8"
        assert pipe.cache_mask_list[0].dtype == torch.bool and not pipe.cache_mask_list[0].any()

        # a written prefix (codes 0x38 = 1.0, scale 2) survives the pipeline's growth loop
        for cache in pipe.kv_cache:
            cache["k"][:, :10].view(torch.uint8).fill_(0x38)
            cache["k_scale"][:, :10].fill_(2.0)
        pipe.cache_valid_len = 10
        pipe._ensure_kv_cache_capacity(64)
        for cache in pipe.kv_cache:
            assert cache["k"].dtype == torch.float8_e4m3fn and cache["k"].shape[1] == 64
            assert (cache["k"][:, :10].view(torch.uint8) == 0x38).all()
            assert (cache["k_scale"][:, :10] == 2.0).all()

        audit = pipe.storage_audit()
        assert audit["int8_kv"] is False and audit["kv_storage_format"] == "fp8"
        per_layer = _fp8_bytes(B, 64, H, D)
        assert audit["gpu_kv_storage_bytes"] == 3 * per_layer
        assert audit["codec_stats"] == [{}, {}, {}]
        assert audit["gpu_kv_peak_working_bytes_upper_bound"] == 3 * per_layer
        for row in audit["kv_storage_layers"]:
            assert set(row) == AUDIT_KEYS
            assert row["storage_dtypes"] == ["torch.float32", "torch.float8_e4m3fn"]
    finally:
        hook.uninstall()
    assert Pipeline.__dict__["_initialize_kv_cache"] is init0


def test_other_formats_stay_on_the_reference_functions():
    storage, int8_kv, Pipeline = make_reference()
    st = pkg_module("kv_cache_storage")
    audit0 = storage.cache_storage_audit
    hook = st.install_fp8_kv_storage(storage, pipeline_cls=Pipeline, int8_kv_module=int8_kv)
    try:
        for mode, code_dtype in (("int8", torch.int8), ("none", torch.bfloat16)):
            pipe = Pipeline(args_for(mode))
            pipe._initialize_kv_cache(1, 8, torch.bfloat16, "cpu")
            assert pipe.kv_cache[0]["k"].dtype == code_dtype
            assert storage.cache_format(pipe.kv_cache[0]) == mode
            assert pipe.storage_audit()["kv_storage_layers"][0] == audit0(pipe.kv_cache[0])
        assert hook.stats["fp8_allocations"] == 0
    finally:
        hook.uninstall()


def test_compressed_storage_checks_apply_to_fp8():
    """The pipeline's refusal of CPU phase-swap offload for quantized
    storage (causal_ar.py:555-557) holds for FP8, and a refused allocation
    leaves the INT8 module and the pipeline flag restored."""
    storage, int8_kv, Pipeline = make_reference()
    st = pkg_module("kv_cache_storage")
    make0 = int8_kv.make_int8_kv_block
    hook = st.install_fp8_kv_storage(storage, pipeline_cls=Pipeline, int8_kv_module=int8_kv)
    try:
        pipe = Pipeline(args_for("fp8", interactive_kv_cache_layerwise_cpu_offload=True))
        with pytest.raises(ValueError, match="PhaseSwappedKVCache"):
            pipe._initialize_kv_cache(1, 8, torch.bfloat16, "cpu")
        assert int8_kv.make_int8_kv_block is make0 and pipe.int8_kv_storage is False
    finally:
        hook.uninstall()


def test_audit_counts_storages_once_and_reads_codec_stats():
    st = pkg_module("kv_cache_storage")
    kvc = pkg_module("fp8_kv_cache")
    cache = kvc.make_fp8_kv_block(1, 16, 3, 128, device="cpu")
    row = st.cache_storage_audit(cache)
    assert set(row) == AUDIT_KEYS and row["storage_format"] == "fp8"
    assert row["gpu_storage_bytes"] == row["peak_working_bytes"] == _fp8_bytes(1, 16, 3, 128)
    assert row["codec_stats"] == {}
    # views of one allocation count once, at the allocation's size
    base = torch.empty(2, 1, 16, 3, 128, dtype=torch.float8_e4m3fn)
    shared = {"k": base[0], "v": base[1], "k_scale": cache["k_scale"], "v_scale": cache["v_scale"]}
    assert st.cache_storage_audit(shared)["gpu_storage_bytes"] == _fp8_bytes(1, 16, 3, 128)
    cache["kv_codec_stats"] = {"peak_working_bytes": 10 ** 9, "note": 1}
    row = st.cache_storage_audit(cache)
    assert row["peak_working_bytes"] == 10 ** 9 and row["codec_stats"]["note"] == 1
    with pytest.raises(ValueError):
        st.install_fp8_kv_storage(make_reference()[0], pipeline_cls=object)
