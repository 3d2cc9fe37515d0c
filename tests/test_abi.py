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


def test_reference_symbol_names_are_kept():
    # the launcher names the reference's kernel_library! blocks bind (gguf/ffi.rs:846-938, 90-147, 227-276)
    L = qmm.lib()
    for t in ("q8_0", "q4_k", "q6_k"):
        for o in ("f32", "f16", "bf16"):
            assert hasattr(L, f"launch_mmvq_gguf_{t}_{o}_plain")
        assert hasattr(L, f"launch_mmvq_gguf_{t}_moe")
    for n in ("launch_moe_dispatch", "launch_moe_weighted_reduce_flat", "launch_moe_weighted_reduce_flat_bf16",
              "launch_moe_weighted_reduce_flat_f16_input", "launch_moe_weighted_reduce_flat_bf16_input"):
        assert hasattr(L, n)
    # the Q8_1 quantizers are deliberately absent: this library's matvecs read Q8_K / Q8_0 blocks
    assert not hasattr(L, "launch_mmvq_gguf_quantize_q8_1_f32")


def test_build_id():
    bid = qmm.build_id()
    assert bid.startswith("qmm-gfx950-")


def test_bad_arguments_are_rejected_before_any_launch():
    L = qmm.lib()
    L.qmm_clear_error()
    # kx_padded not a multiple of 256: nothing launched, an error recorded
    L.launch_mmvq_gguf_quantize_q8k_f32(None, None, 300, 300, 1, None)
    assert "multiple of 256" in qmm.last_error()
    with pytest.raises(qmm.QmmError):
        qmm.check()
    assert qmm.last_error() == ""
    L.launch_mmvq_gguf_q4_k_f32_plain(None, None, None, 100, 8, 1, 8, 1, None)
    assert "ncols_x" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_mmvq_gguf_q4_k_f32_plain(None, None, None, 256, 8, 1, 8, 33, None)  # Q4_K takes up to 32 rows
    assert "b_size" in qmm.last_error()
    L.qmm_clear_error()
    L.launch_indexed_moe_forward_q4k_q8k(None, None, None, None, 8, 256, 2, 2, 256, 3, None)
    assert "input_dim1" in qmm.last_error()
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


def test_host_library_exports_its_header():
    import ctypes as C
    L = C.CDLL(qmm.HOST_LIB_PATH)
    names = qmm.declared_symbols(qmm.HEADERS[1])
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
