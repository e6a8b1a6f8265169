"""The C ABI library: loads, exports every declared symbol, host-only logic.

No compute calls here (no GPU on the CPU test host): only entry points that
return before touching HIP - size queries, argument validation, empty inputs.
"""

from __future__ import annotations

import ctypes
import re

import pytest

from cuda_force_amd import _lib


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_function_is_exported_and_bound(lib):
    declared = _lib.declared_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/cudaforge_hip.h but not exported"
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures out of step with the header"


def test_every_header_function_cites_a_reference_interface_or_says_it_has_none():
    text = _lib.HEADER.read_text(encoding="utf-8")
    for name in _lib.declared_functions():
        decl = re.search(rf"^[a-z_0-9 ]+\**\s*{name}\(", text, re.M).start()
        comment = text[max(0, text.rfind("/*", 0, decl)) : decl]
        flat = " ".join(comment.replace("*", " ").split())
        assert re.search(r"\.(cuh|cu|cpp|py|hpp):\d+|no counterpart in the reference", flat), (
            f"{name} has no reference citation"
        )


def test_the_block_size_and_scale_count(lib):
    text = _lib.HEADER.read_text(encoding="utf-8")
    assert re.search(r"#define CF_QUANT_BLOCK_SIZE 64\b", text)
    assert [lib.cf_quant_scale_count(n) for n in (-5, 0, 1, 64, 65, 4096 * 4096)] == [0, 0, 1, 1, 2, 262144]


def test_workspace_queries(lib):
    assert lib.cf_lora_workspace_bytes(8, 16) == 8 * 16 * 4
    assert lib.cf_lora_workspace_bytes(0, 16) == 0
    assert lib.cf_reduce_sum_workspace_bytes(0) == 0
    assert lib.cf_reduce_sum_workspace_bytes(1) == 4
    assert lib.cf_reduce_sum_workspace_bytes(1 << 30) == 4096 * 4
    assert lib.cf_lora_backward_workspace_bytes(8192, 4096, 4096, 16) >= 8192 * 16 * 4
    assert lib.cf_abi_version() == 1


def test_empty_inputs_return_ok_without_touching_the_device(lib):
    null = ctypes.c_void_p(0)
    assert lib.cf_quantize_int8(null, _lib.CF_F32, null, null, 0, null) == _lib.CF_OK
    assert lib.cf_dequantize_int8(null, null, null, _lib.CF_F32, -1, null) == _lib.CF_OK
    assert lib.cf_rmsnorm(null, null, null, _lib.CF_BF16, 0, 4096, 1e-6, null) == _lib.CF_OK
    assert lib.cf_softmax(null, _lib.CF_F32, null, _lib.CF_F32, 5, 0, null) == _lib.CF_OK
    assert lib.cf_softmax_scaled(null, _lib.CF_BF16, null, _lib.CF_BF16, 0, 512, 0.5, 512, null) == _lib.CF_OK
    fake = ctypes.c_void_p(0x1000)  # rejected before any launch
    assert lib.cf_softmax_scaled(fake, _lib.CF_BF16, fake, _lib.CF_BF16, 4, 4, 0.5, -1, null) == \
        _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_lora_linear(null, null, null, null, null, null, _lib.CF_BF16, 0, 8, 8, 2, 1.0, null) == _lib.CF_OK


def test_invalid_arguments_are_reported_not_thrown(lib):
    null = ctypes.c_void_p(0)
    status = lib.cf_quantize_int8(null, _lib.CF_F32, null, null, 10, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"null pointer" in lib.cf_last_error()
    # Any rank is taken (large ranks run the generic path); an unfused shape
    # without the xa workspace is an argument error raised before any launch.
    status = lib.cf_lora_linear(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                ctypes.c_void_p(16), ctypes.c_void_p(16), null, _lib.CF_F32,
                                8, 8, 8, 128, 1.0, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"xa_out" in lib.cf_last_error()
    status = lib.cf_lora_linear(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                ctypes.c_void_p(16), ctypes.c_void_p(16), null, _lib.CF_F16,
                                8, 8, 8, 4, 1.0, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"float16" in lib.cf_last_error()
    status = lib.cf_reduce_sum(ctypes.c_void_p(16), _lib.CF_F32, ctypes.c_void_p(16), 1000,
                               null, 0, 0, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"workspace" in lib.cf_last_error()
    # The LoRA workspace. bf16: an 8-byte flag per 256-row tile (the block
    # rounded up to 256 bytes) plus 8 KiB per tile for the fused kernel's
    # shared x @ a (0 for rank 0, odd ranks and shapes the fused kernel does
    # not take). fp32: 0 for shapes the fp32 MFMA kernel does not take. One
    # smaller than asked for is rejected before any launch.
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 32, 1024, 1024, 8) == 256 + 8192
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 8192, 4096, 4096, 16) == 256 + 32 * 8192
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 8192 * 8 + 1, 4096, 4096, 16) == 2304 + 257 * 8192
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 32, 1024, 1024, 0) == 0
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 32, 1024, 1024, 7) == 0
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 32, 1000, 1024, 8) == 0
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 32, 1024, 1020, 8) == 0
    bf16_bytes = lib.cf_lora_linear_ws_bytes(_lib.CF_BF16, 32, 1024, 1024, 8)
    status = lib.cf_lora_linear_ws(p4k := ctypes.c_void_p(4096), p4k, p4k, p4k, p4k, null, _lib.CF_BF16,
                                   32, 1024, 1024, 8, 0.5, p4k, bf16_bytes - 16, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"workspace" in lib.cf_last_error()
    status = lib.cf_lora_linear_ws(p4k, p4k, p4k, p4k, p4k, null, _lib.CF_BF16, 32, 1024, 1024, 8, 0.5,
                                   ctypes.c_void_p(4096 + 8), bf16_bytes, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"aligned" in lib.cf_last_error()
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_F32, 32, 1022, 1024, 8) == 0
    assert lib.cf_lora_linear_ws_bytes(_lib.CF_F32, 32, 1024, 1024, 17) == 0
    nbytes = lib.cf_lora_linear_ws_bytes(_lib.CF_F32, 32, 1024, 1024, 8)
    assert nbytes >= 2 * 32 * 1024 * 4
    p = ctypes.c_void_p(4096)
    status = lib.cf_lora_linear_ws(p, p, p, p, p, null, _lib.CF_F32, 32, 1024, 1024, 8, 0.5, p,
                                   nbytes - 256, null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"workspace" in lib.cf_last_error()
    status = lib.cf_lora_linear_ws(p, p, p, p, p, null, _lib.CF_F16, 32, 1024, 1024, 8, 0.5, null, 0,
                                   null)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"float16" in lib.cf_last_error()


def test_sticky_error_classification(lib):
    # hipErrorIllegalAddress (700) poisons the context; hipErrorInvalidValue (1) does not.
    assert lib.cf_hip_error_is_sticky(700) == 1
    assert lib.cf_hip_error_is_sticky(1) == 0


def test_the_error_slot_is_per_thread(lib):
    import threading

    null = ctypes.c_void_p(0)
    lib.cf_quantize_int8(null, _lib.CF_F32, null, null, 10, null)
    seen = {}

    def other():
        seen["msg"] = lib.cf_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == b"no error"
    assert b"null pointer" in lib.cf_last_error()


def test_paged_attention_argument_errors_need_no_device():
    lib = _lib.load()
    null = None
    assert lib.cf_paged_attention(null, null, null, null, null, null, _lib.CF_F32, 0, 4, 2, 32, 4, 1,
                                  1.0, null, 0, null) == _lib.CF_OK
    assert lib.cf_paged_attention(null, null, null, null, null, null, _lib.CF_F32, 1, 3, 2, 32, 4, 1,
                                  1.0, null, 0, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_paged_attention(null, null, null, null, null, null, _lib.CF_F32, 1, 2, 2, 2048, 4, 1,
                                  1.0, null, 0, null) == _lib.CF_ERR_INVALID_ARGUMENT


def test_time_next_launch_takes_both_events_or_neither(lib):
    null = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: rejected before use
    assert lib.cf_time_next_launch(fake, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_time_next_launch(null, fake) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_time_next_launch(null, null) == _lib.CF_OK


def test_an_entry_point_that_launches_nothing_disarms_the_timing_events(lib):
    """Armed events belong to the next operator call: one that returns before
    launching (empty input, invalid argument) must not leave them for a later,
    unrelated launch. The fake handles are never used: nothing launches."""
    null = ctypes.c_void_p(0)
    fake_start, fake_stop = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000)
    assert lib.cf_time_next_launch_armed() == 0
    calls = [
        lambda: lib.cf_rmsnorm(null, null, null, _lib.CF_BF16, 0, 4096, 1e-6, null),         # empty
        lambda: lib.cf_reduce_sum(null, _lib.CF_F32, null, 0, null, 0, 1, null),              # empty
        lambda: lib.cf_quantize_int8(null, _lib.CF_F32, null, null, 10, null),                # null pointer
        lambda: lib.cf_softmax(null, _lib.CF_F32, null, 7, 4, 4, null),                       # bad dtype
        lambda: lib.cf_matmul_tensor_core(null, null, null, 4, 5, 4, null, 0, null),          # unsupported
        lambda: lib.cf_lora_backward(null, null, null, null, null, null, _lib.CF_F32, 8, 8, 8, 0, 1.0,
                                     null, 0, null),                                          # rank 0
    ]
    for call in calls:
        assert lib.cf_time_next_launch(fake_start, fake_stop) == _lib.CF_OK
        assert lib.cf_time_next_launch_armed() == 1
        call()
        assert lib.cf_time_next_launch_armed() == 0
    # Runtime calls are not operator launches: they leave the events armed.
    assert lib.cf_time_next_launch(fake_start, fake_stop) == _lib.CF_OK
    assert lib.cf_pool_backend_name(_lib.CF_POOL_HOST) == b"host"
    assert lib.cf_time_next_launch_armed() == 1
    assert lib.cf_time_next_launch(null, null) == _lib.CF_OK
    assert lib.cf_time_next_launch_armed() == 0


def test_grouped_quantisation_host_checks(lib):
    null = ctypes.c_void_p(0)
    # Nothing to do: returns before touching anything.
    assert lib.cf_quantize_int8_group(null, _lib.CF_F32, null, null, null, 0, null) == _lib.CF_OK
    assert lib.cf_dequantize_int8_group(null, null, null, _lib.CF_BF16, null, -3, null) == _lib.CF_OK
    # Missing arrays are argument errors.
    assert lib.cf_quantize_int8_group(null, _lib.CF_F32, null, null, null, 2, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_dequantize_int8_group(null, null, null, _lib.CF_F32, null, 1, null) == _lib.CF_ERR_INVALID_ARGUMENT
    # Empty members are skipped (no launch, no pointer check); a null pointer
    # in a non-empty member is rejected before any launch.
    ptrs = _lib.pointer_array([0, 0])
    counts = _lib.int64_array([0, -1])
    assert lib.cf_quantize_int8_group(ptrs, _lib.CF_F32, ptrs, ptrs, counts, 2, null) == _lib.CF_OK
    counts = _lib.int64_array([0, 64])
    assert lib.cf_quantize_int8_group(ptrs, _lib.CF_F32, ptrs, ptrs, counts, 2, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert b"tensor 1" in lib.cf_last_error()
    assert lib.cf_dequantize_int8_group(ptrs, ptrs, ptrs, _lib.CF_F32, counts, 2, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_quantize_int8_group(ptrs, 7, ptrs, ptrs, counts, 2, null) == _lib.CF_ERR_UNSUPPORTED


def test_stream_bytes_host_checks(lib):
    null = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: rejected before any launch
    assert lib.cf_stream_bytes(null, null, 0, 4, null) == _lib.CF_OK
    assert lib.cf_stream_bytes(fake, fake, 16384, 3, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(null, null, 16384, -1, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(null, fake, 16384, 0, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(fake, fake, 1000, 4, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(null, fake, 16384, 4, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(null, null, 16384, -3, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(null, fake, 16384, -6, null) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_stream_bytes(null, fake, 1 << 32, -2, null) == _lib.CF_ERR_INVALID_ARGUMENT


def test_attention_products_host_checks(lib):
    """The causal attention products reject what they have no kernel for
    before any launch: empty sizes are no-ops, fp32, a head size outside
    32/64/96/128 or a sequence length that is not a multiple of 8 are
    CF_ERR_UNSUPPORTED, null or misaligned tensors CF_ERR_INVALID_ARGUMENT."""
    null = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)
    odd = ctypes.c_void_p(0x1008)
    for name in ("cf_attention_scores_causal", "cf_attention_pv_causal"):
        fn = getattr(lib, name)
        assert fn(null, null, null, _lib.CF_BF16, 0, 512, 32, 128, null) == _lib.CF_OK
        assert fn(null, null, null, _lib.CF_BF16, 8, 0, 32, 128, null) == _lib.CF_OK
        assert fn(null, fake, fake, _lib.CF_BF16, 8, 512, 32, 128, null) == _lib.CF_ERR_INVALID_ARGUMENT
        assert fn(fake, fake, fake, _lib.CF_F32, 8, 512, 32, 128, null) == _lib.CF_ERR_UNSUPPORTED
        assert fn(fake, fake, fake, _lib.CF_BF16, 8, 512, 32, 80, null) == _lib.CF_ERR_UNSUPPORTED
        assert fn(fake, fake, fake, _lib.CF_BF16, 8, 500, 32, 128, null) == _lib.CF_ERR_UNSUPPORTED
        assert fn(fake, odd, fake, _lib.CF_BF16, 8, 512, 32, 128, null) == _lib.CF_ERR_INVALID_ARGUMENT
        assert b"16-byte aligned" in lib.cf_last_error()
        assert fn(fake, fake, fake, _lib.CF_BF16, 1, 32768, 2, 128, null) == _lib.CF_ERR_INVALID_ARGUMENT
        assert b"32-bit offsets" in lib.cf_last_error()
