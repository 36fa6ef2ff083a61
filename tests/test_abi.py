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
    # rows * (Kpad + Npad + 1) + min(rows, 8) * (Kpad / 128) * Npad
    assert lib.exl3_linear_workspace_size(1, 4096, 14336) == 1 * (4096 + 14336 + 1) + 32 * 14336
    assert lib.exl3_linear_workspace_size(-1, 128, 128) == -1
    assert lib.exl3_moe_workspace_size(4, 256, 200, 2, 0) == 0
    size = lib.exl3_moe_workspace_size(4, 256, 200, 2, 3)
    a, hpad, ipad = 8, 256, 256
    ints = 4 + (a + 3) // 4 * 4 + 4 * a + a * max(hpad, ipad) // 128
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
