"""CPU checks of the C-ABI boundary: the library loads without a GPU, exports
every function include/ti.h declares, and reports errors through ti_last_error."""
import ctypes as C
import os
import subprocess

import pytest

from tabinfer_amd import abi


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    names = abi.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_nm_agrees_with_header():
    out = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH], stdout=subprocess.PIPE, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(abi.header_functions()) <= exported


def test_every_declared_function_has_a_binding():
    # every entry point of ti.h is callable from Python with declared argtypes
    names = set(abi.header_functions()) - {"ti_last_error"}
    assert names <= set(abi.SIGS), sorted(names - set(abi.SIGS))


def test_no_device_is_a_clean_error():
    if abi.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(abi.TIError) as e:
        abi.Ctx(0)
    assert e.value.code == abi.TI_ERR_NO_DEVICE
    assert "no HIP device" in str(e.value)


def test_null_context_is_rejected():
    lib = abi.lib()
    assert lib.ti_sync(None) == abi.TI_ERR_INVALID
    assert b"null context" in lib.ti_last_error()
    assert lib.ti_gemv_q4_q8(None, None, None, None, None, None, 1, 32, 0) == abi.TI_ERR_INVALID
    assert lib.ti_graph_destroy(None) == 0
