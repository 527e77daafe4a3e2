"""The C ABI: libncmhip.so loads, exports every function include/ncm_hip.h
declares, and reports errors through the record mode instead of exiting."""
import ctypes
import os

import numpy as np
import pytest

import ncmhip


def test_library_built():
    assert os.path.exists(ncmhip.LIB_PATH), "run __graft_entry__.build() first"


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(ncmhip.LIB_PATH)
    declared = ncmhip.header_functions()
    assert "linear_fwd" in declared and "vq_argmin" in declared
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the whole header
    assert sorted(ncmhip._SIGS) == sorted(declared)


def test_tape_library_exports_the_reference_prototypes():
    """libncmhip_tape.so exports every function include/ncm_hip_tape.h
    declares (the reference's tape names, ncm.h:192-195, 468-522), each one
    resolved against libncmhip.so."""
    import re
    header = open(os.path.join(os.path.dirname(ncmhip.HERE), "include", "ncm_hip_tape.h")).read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    declared = re.findall(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\(", header, flags=re.M)
    assert {"tape_new", "t_linear", "t_ce", "tape_backward", "t_qkvsplit"} <= set(declared)
    lib = ctypes.CDLL(os.path.join(ncmhip.HERE, "libncmhip_tape.so"))
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing


def test_bad_arguments_are_errors_not_exits():
    ncmhip.load()
    with pytest.raises(ncmhip.NcmError, match="bad shape"):
        ncmhip.linear_fwd(None, None, None, None, 4, 0, 8)
    with pytest.raises(ncmhip.NcmError, match="unknown activation"):
        ncmhip.load().linear_fwd_ep(None, None, None, None, None, 4, 4, 4, 9)
        ncmhip.check()
    with pytest.raises(ncmhip.NcmError, match="D=5000"):
        ncmhip.vq_argmin(None, None, None, 10, 16, 5000)
    with pytest.raises(ncmhip.NcmError, match="bad shape"):
        ncmhip.argmax_rows(None, None, 1, 0)


def test_host_argmax_row_matches_reference_semantics():
    lib = ncmhip.load()
    for arr, want in (([1, 3, 3, 2], 1), ([np.nan, 3, 4], 0), ([1, np.nan, 4, 4], 2)):
        a = np.array(arr, np.float32)
        assert lib.argmax_row(a.ctypes.data, a.size) == want


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_device_is_a_clean_error():
    with pytest.raises(ncmhip.NcmError):
        ncmhip.init(0)


def test_code_objects_have_no_scalar_stores():
    """Every embedded gfx950 code object writes through vector memory only:
    no scalar-cache stores, atomics, write-backs or discards."""
    import glob
    import re
    import subprocess
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    cos = glob.glob(os.path.join(ncmhip.HERE, "build", "*.co"))
    if not cos or not os.path.exists(objdump):
        pytest.skip("code objects or llvm-objdump not available")
    bad = re.compile(r"\bs_(store|atomic|buffer_store|buffer_atomic|dcache_wb|dcache_discard|scratch_store)")
    for co in cos:
        text = subprocess.run([objdump, "-d", co], check=True, capture_output=True, text=True).stdout
        hits = [ln for ln in text.splitlines() if bad.search(ln)]
        assert not hits, (co, hits[:3])
