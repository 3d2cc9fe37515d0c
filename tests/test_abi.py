"""CPU tests of the C ABI boundary: the library loads, exports every symbol the headers declare, carries a
build id (kernel_library.rs:288-297), and rejects arguments it cannot serve without touching a GPU."""
import ctypes
import subprocess

import pytest

import qmm


def test_library_exports_every_declared_symbol():
    L = qmm.lib()
    names = qmm.declared_symbols(qmm.HEADERS[0])
    assert len(names) >= 30, names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    nm = subprocess.run(["nm", "-D", "--defined-only", qmm.LIB_PATH], capture_output=True, text=True, check=True).stdout
    for n in names:
        assert f" {n}\n" in nm, n


# argument kinds of the ctypes prototypes derived from include/inferencequant.h, as the fixture names them
_KIND = {ctypes.c_void_p: "ptr", ctypes.c_int: "i32", ctypes.c_int32: "i32", ctypes.c_int64: "i64",
         ctypes.c_uint32: "u32", ctypes.c_float: "f32", ctypes.c_bool: "bool"}


def test_reference_symbols_bind_unchanged():
    """Every kernel-library symbol the reference declares for the weight types served here (tests/golden/
    reference_abi.json, read from gguf/ffi.rs and inference-nn/src/cuda/ffi.rs by make_reference_abi.py) is exported
    with the same argument kinds, count and return type, so its kernel_library! blocks bind with no edit."""
    import json
    import os
    ref = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_abi.json")))
    assert len(ref) >= 120
    L = qmm.lib()
    protos = qmm.prototypes()
    problems = []
    for name, sig in ref.items():
        if not hasattr(L, name) or name not in protos:
            problems.append(f"{name}: not exported / declared")
            continue
        restype, argtypes = protos[name]
        kinds = [_KIND[a] for a in argtypes]
        if kinds != sig["args"]:
            problems.append(f"{name}: arguments {kinds} against the reference's {sig['args']}")
        ret = "void" if restype is None else "i32" if restype is ctypes.c_int else str(restype)
        if ret != sig["ret"]:
            problems.append(f"{name}: returns {ret} against the reference's {sig['ret']}")
    assert not problems, problems
    # every call sequence of SURVEY's boundary has its entries: decode, prefill, GLU requantization, indexed and fused
    # MoE, dispatch / reduce, gather
    for n in ("launch_mmvq_gguf_quantize_q8_1_f32", "launch_mmq_quantize_q8_1_DS4", "launch_mmq_quantize_glu_q8_1_D4",
              "launch_indexed_moe_forward_q4k_q8_1", "launch_moe_gemv_fused_gate_up_q4k_q8_1",
              "launch_moe_gemv_down_aggregate_q6k_q8_1", "launch_gather_rows_u8", "launch_moe_dispatch"):
        assert n in ref, n


def test_build_id():
    bid = qmm.build_id()
    assert bid.startswith("qmm-gfx950-")


def test_bad_arguments_are_rejected_before_any_launch():
    L = qmm.lib()
    L.qmm_clear_error()
    # kx_padded not a multiple of 256: nothing launched, an error recorded
    L.launch_mmvq_gguf_quantize_q8_1_f32(None, None, 300, 300, 1, None)
    assert "multiple of 256" in qmm.last_error()
    with pytest.raises(qmm.QmmError):
        qmm.check()
    assert qmm.last_error() == ""
    L.launch_mmvq_gguf_q4_k_f32_plain(None, None, None, 100, 8, 8, 8, 1, None)
    assert "ncols_x" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmvq_gguf_q4_k_f32_plain(None, None, None, 256, 8, 8, 8, 33, None)  # Q4_K takes up to 32 rows
    assert "b_size" in qmm.last_error()
    L.qmm_clear_error()
    # slots: stride_col_y counts 32-value Q8_1 blocks and must hold whole 256-value slots
    L.launch_mmvq_gguf_q4_k_f32_plain(None, None, None, 256, 8, 12, 8, 1, None)
    assert "stride_col_y" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_indexed_moe_forward_q4k_q8_1(None, None, None, None, 8, 256, 2, 2, 256, 3, None)
    assert "input_dim1" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_moe_gemv_fused_gate_up_q4k_q8_1(None, None, None, None, None, 8, 256, 1, 2, 256, 1, None)
    assert "moe_gemv_fused_gate_up" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_moe_gemv_down_aggregate_q8_0_q8_1(None, None, None, None, None, 8, 256, 1, 2, 300, None)
    assert "k_padded" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_gather_rows_u8(None, None, None, 0, 1, 1, None)
    assert "gather_rows_u8" in qmm.last_error()
    L.qmm_clear_error()
    rc = L.launch_moe_weighted_reduce_flat(None, None, None, 1, 1, 0, None)
    assert rc != 0 and "topk" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_dequantize_q4_k_f32(None, None, 300, None)
    assert "multiple of 256" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_get_rows_q8_0(None, None, None, 40, 34, 1, None)
    assert "ne00" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmvq_gguf_q8_0_f32_exact(None, None, None, 64, 4, 9, None)
    assert "b_size" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmq_quantize_q8_1_D4(None, None, None, 0, 300, 300, 300, 300, 300, 1, 1, 1, None)
    assert "multiple of 256" in qmm.last_error()
    L.qmm_clear_error()
    # the `_q8k` prefill entries
    L.launch_mmq_quantize_q8k(None, None, None, 0, 300, 300, 300, 300, 300, 1, 1, 1, None)
    assert "mmq_quantize_q8k" in qmm.last_error() and "multiple of 256" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmq_quantize_glu_q8k_f32(None, None, None, None, 256, 256, 256, 1, 5, None)
    assert "activation" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmq_gguf_q4_k_q8k(None, 8, None, None, 256, 8, 1, 1, 8, 0, 256, 0, 64, 0, None)
    assert "16-byte aligned" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmq_gguf_q5_k_q8k(None, None, None, None, 300, 8, 1, 1, 8, 0, 256, 0, 64, 0, None)
    assert "ncols_x" in qmm.last_error()
    L.qmm_clear_error()


def test_host_library_exports_its_header():
    import ctypes as C
    L = C.CDLL(qmm.HOST_LIB_PATH)
    names = qmm.declared_symbols(qmm.HEADERS[1])
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
