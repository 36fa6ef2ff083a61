"""The C-ABI boundary on the CPU (no GPU calls): libvllm_mi355x.so loads,
exports every function include/vllm_mi355x.h declares, the ctypes table
mirrors the header, the operator libraries register the reference's
schemas, and the host-only size functions and checks behave."""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vllm_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_boundary():
    names = set(declared_functions())
    for name in ("exl3_linear_out", "exl3_moe_out", "exl3_decode", "marlin_moe_gemm",
                 "marlin_moe_act", "moe_align_block_size", "moe_sum", "marlin_dequant"):
        assert name in names


def test_library_exports_every_declared_symbol():
    from vllm_mi355x import _native
    lib = ctypes.CDLL(_native.LIBRARY_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(_native.SIGNATURES)
    assert _native.load().vllm_mi355x_abi_version() == _native.ABI_VERSION


def test_workspace_size_functions():
    from vllm_mi355x import _native
    lib = _native.load()
    # max(small-M partials: min(rows, 8) * splits * Npad at the automatic
    # split count, large-M: rows * (Kpad + 1) above 32 rows)
    # 4096 x 14336: 2 input blocks per workgroup, 16 splits
    assert lib.exl3_linear_workspace_size(1, 4096, 14336) == 1 * 16 * 14336
    # 8192 x 28672: 8 blocks, 8 splits; 1024 rows take the large-M term
    assert lib.exl3_linear_workspace_size(8, 8192, 28672) == 8 * 8 * 28672
    assert lib.exl3_linear_workspace_size(1024, 8192, 28672) == 1024 * 8193
    assert lib.exl3_linear_workspace_size(32, 256, 256) == 8 * 2 * 256
    assert lib.exl3_linear_workspace_size(-1, 128, 128) == -1
    assert lib.exl3_linear_prefill_rows() == 32
    assert lib.exl3_moe_workspace_size(4, 256, 200, 2, 0) == 0
    size = lib.exl3_moe_workspace_size(4, 256, 200, 2, 3)
    a, hpad, ipad = 8, 256, 256
    ints = 4 + (a + 3) // 4 * 4 + 4 * a + a * max(hpad, ipad) // 128 + a
    assert size == a * (hpad + 3 * ipad) + ints
    assert lib.exl3_moe_workspace_size(4, 0, 200, 2, 3) == -1


def test_marlin_host_checks_reject_bad_shapes():
    from vllm_mi355x import _native
    lib = _native.load()
    # K not a multiple of 128: rejected before any launch
    rc = lib.marlin_moe_gemm(0, 0, 1, 136, 0, 0, 1, 0, 8, 0, 1, 0, 0, 1, 1, 136, 64, 8, 0, 1, 0,
                             0, 0, 0, 0, 0)
    assert rc == 1 and b"K % 128" in lib.vllm_mi355x_last_error()
    rc = lib.moe_align_block_size(0, 4, 0, 8, 0, 0, 64, 0, 8, 0, 0)
    assert rc == 1 and b"num_experts" in lib.vllm_mi355x_last_error()


def test_operator_schemas_register():
    from vllm_mi355x.kernels.exl3 import ops
    from vllm_mi355x.kernels.marlin_moe import extension
    ops.ensure_extension()
    extension.require_extension()
    schema = torch._C._dispatch_find_schema_or_throw("_exl3_C::moe_out_v2", "").schema()
    assert [a.name for a in schema.arguments][6:8] == ["intermediate_size", "bits_x2"]
    info = __import__("vllm_mi355x.kernels.marlin_moe._C", fromlist=["build_info"]).build_info()
    assert info["abi_version"] == 1 and info["prefill_schedule_version"] == 2


def test_block_size_and_split_choice():
    from vllm_mi355x.kernels.marlin_moe.fused import choose_block_size, choose_w13_ksplit
    from vllm_mi355x.kernels.moe.align import align_sizes
    assert choose_block_size(1, 8, 128) == 8
    assert choose_block_size(256, 8, 128) in (32, 64)
    assert choose_block_size(2048, 8, 128) == 64
    assert align_sizes(8, 128, 8) == (64, 8)
    assert align_sizes(2048, 128, 64) == (2048 + 128 * 63, (2048 + 128 * 63 + 63) // 64)
    ks = choose_w13_ksplit(8, 1536, 2048, 8)
    assert 1 <= ks and (2048 // 128) % ks == 0 and (2048 // 128) // ks >= 4


def test_linear_row_chunk_reaches_the_prefill_gemm():
    """The reference's fixed 8M-float dense scratch (ops.py:31-33) holds
    more rows per chunk than the small-M threshold at the prefill shapes,
    so exl3_linear runs prefills on the large-M GEMM."""
    from vllm_mi355x.kernels.exl3 import ops
    assert ops.linear_row_chunk(8192, 28672) > 32
    assert ops.linear_row_chunk(7168, 18432) > 32
    assert ops.linear_row_chunk(4096, 14336) > 32
    assert torch.ops._exl3_C.linear_prefill_applies(33, 4096, 4096, 8, 2)
    assert not torch.ops._exl3_C.linear_prefill_applies(32, 4096, 4096, 8, 2)


def _runtime_build_info(abi_version):
    cuda = torch.version.cuda
    major, minor = (int(v) for v in cuda.split(".")[:2]) if cuda else (0, 0)
    return {"abi_version": abi_version, "torch_version": torch.__version__.split("+")[0],
            "cuda_version": major * 1000 + minor * 10,
            "cxx11_abi": int(torch._C._GLIBCXX_USE_CXX11_ABI)}


def _compare_build_info(built, abi_version):
    for key, expected in _runtime_build_info(abi_version).items():
        actual = built.get(key)
        if key == "cuda_version" and isinstance(actual, int):
            actual, expected = actual // 1000, expected // 1000
        assert actual == expected, key


def test_reference_loader_accepts_the_exl3_library():
    """The reference's _validate_extension (vllm_sm80/kernels/exl3/ops.py:
    193-240), replayed: build_info keys, every operator it calls, and the
    two custom classes, which exist and raise when constructed."""
    from vllm_mi355x.kernels.exl3 import _C, ops
    ops.ensure_extension()
    _compare_build_info(_C.build_info(), 3)
    for name in ("linear_out", "linear_out_splitk", "moe_out", "moe_out_v2", "moe_out_prefill",
                 "ple_decode_out", "ple_read_rows", "linear_workspace_size", "linear_splitk_splits",
                 "moe_workspace_size", "moe_workspace_size_v2", "moe_workspace_size_prefill"):
        torch._C._dispatch_find_schema_or_throw(f"_exl3_C::{name}", "")
    for name in ("PleHostReader", "EngramHostFetch"):
        getattr(torch.classes._exl3_C, name)
    with pytest.raises(RuntimeError, match="PleHostReader"):
        torch.classes._exl3_C.PleHostReader(0, torch.zeros(1), torch.zeros(1), 0, 0, 0, 0,
                                            torch.zeros(1), torch.zeros(1), 0, 0, 0)
    with pytest.raises(RuntimeError, match="EngramHostFetch"):
        torch.classes._exl3_C.EngramHostFetch(0, 0, 0, 0, 0, *[torch.zeros(1)] * 5, 0, 0, 0, 0, 0)
    # the operators the reference's loader registers fakes for
    for name in ("linear_out", "linear_out_splitk", "moe_out", "moe_out_v2", "moe_out_prefill",
                 "ple_decode_out"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"_exl3_C::{name}", "CUDA"), name


def test_reference_loader_accepts_the_marlin_library():
    """The reference's Marlin _validate_extension and prefill_tile_op
    (vllm_sm80/kernels/marlin_moe/extension.py:19-43, :56-81, :86-112),
    replayed: build_info, argument names / types / returns of each
    operator, a CUDA kernel for each, the prefill schedule version."""
    from vllm_mi355x.kernels.marlin_moe import _C, extension
    extension.require_extension()
    _compare_build_info(_C.build_info(), 1)
    expected = {
        "decode_gemm_orig": (
            "a w s sorted eids ntpp topk_w topk n_slots K N w13 rows cfg ctr out",
            "Tensor Tensor Tensor Tensor Tensor Tensor Tensor int int int int bool int int Tensor Tensor",
            "int"),
        "decode_act_orig": ("part ids ksplit n_slots Nh limit h", "Tensor Tensor int int int float Tensor", ""),
    }
    for name, want in expected.items():
        qualified = f"_ampere_marlin_C::{name}"
        schema = torch._C._dispatch_find_schema_or_throw(qualified, "").schema()
        got = (" ".join(a.name for a in schema.arguments), " ".join(str(a.type) for a in schema.arguments),
               " ".join(str(a.type) for a in schema.returns))
        assert got == want, name
        assert torch._C._dispatch_has_kernel_for_dispatch_key(qualified, "CUDA"), name
    assert _C.build_info()["prefill_schedule_version"] == 2
    schema = torch._C._dispatch_find_schema_or_throw("_ampere_marlin_C::prefill_tile_gemm", "").schema()
    assert " ".join(a.name for a in schema.arguments) == (
        "a c_or_none b_q_weight b_bias_or_none b_scales a_scales global_scale "
        "b_zeros_or_none workspace sorted_token_ids expert_ids num_tokens_past_padded "
        "topk_weights moe_block_size top_k mul_topk_weights b_type_id size_m size_n "
        "size_k use_atomic_add use_fp32_reduce is_zp_float thread_k thread_n "
        "blocks_per_sm c_tmp redo")


def test_moe_launch_rows_keeps_offsets_in_32_bits():
    from vllm_mi355x.kernels.exl3 import ops
    rows = ops.moe_launch_rows(7168, 2048, 9)
    assert rows == (2 ** 31 - 1) // (4 * 7168 * 9)
    assert rows * 9 * 7168 * 4 <= 2 ** 31 - 1 < (rows + 1) * 9 * 7168 * 4
    assert ops.moe_launch_rows(100, 300, 8) == (2 ** 31 - 1) // (4 * 384 * 8)
