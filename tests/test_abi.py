"""The C-ABI library loads and exports every function include/mlamoe.h
declares (no GPU needed), and reports errors instead of exiting."""
import ctypes as C
import os
import subprocess

import pytest

import mlamoe


def test_library_built_and_exports_header():
    L = mlamoe.lib()
    names = mlamoe.header_functions()
    assert "mm_moe_forward_dev" in names and "mm_ffn_compute" in names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_exports_only_the_c_abi():
    """Every exported function is declared in the header: no C++ symbols and
    no torch types cross the boundary."""
    out = subprocess.run(["nm", "-D", "--defined-only", mlamoe.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert exported == set(mlamoe.header_functions()), exported ^ set(mlamoe.header_functions())


def test_errors_are_returned_not_fatal():
    L = mlamoe.lib()
    assert L.mm_ctx_sync(None) != 0
    assert b"NULL" in L.mm_last_error()
    h = C.c_void_p()
    st = L.mm_ctx_create(-1, C.byref(h))
    assert st != 0 and h.value is None
    assert L.mm_last_error()


def test_no_gpu_context_fails_loudly():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(mlamoe.MMError):
        mlamoe.Context(0)


@pytest.mark.skipif(not os.path.isdir("/root/reference/include"),
                    reason="the reference tree is not present here")
def test_getp_shim_compiles_against_reference_headers():
    """mla-moe_amd/shim/getp_mlamoe.c implements include/getp.h's warm_up /
    inference / finish on the C-ABI; it must compile against the reference's
    own headers (model.h, getp.h, tokenizer.h) with the reference's C flags."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run(["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                        "-I/root/reference/include", "-I" + os.path.join(root, "include"),
                        os.path.join(root, "mla-moe_amd", "shim", "getp_mlamoe.c")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
