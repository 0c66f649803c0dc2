"""The C-ABI library loads, exports every symbol the header declares, and
refuses bad calls with a reason -- all without touching a GPU."""
import ctypes as C
import subprocess

import ming_dit_amd as m


def test_library_exports_every_header_symbol():
    m.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", m.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    declared = m.header_symbols()
    assert len(declared) >= 20
    missing = [s for s in declared if s not in exported]
    assert missing == [], missing


def test_abi_version():
    assert m.lib().ming_abi_version() == 5


def test_engagement_layout_matches_the_header():
    """The ctypes mirror of ming_engagement has the header's fields in order."""
    import re
    txt = open(m.HEADER).read()
    body = txt[txt.index("typedef struct ming_engagement"):txt.index("} ming_engagement;")]
    names = re.findall(r"int64_t\s+(\w+);", body)
    assert names == [n for n, _ in m.Engagement._fields_]


def test_null_arguments_are_refused_with_a_reason():
    L = m.lib()
    assert L.ming_lin(None, None, None, 0, None, 0, 0, None) == 1
    assert b"null" in L.ming_last_error()
    assert L.ming_rmsnorm(None, None, 0, None, None, 0, 0, 0, 1e-5) == 1
    assert L.ming_qweight_bind_lora(None, 0, 0, 4, None, None, 1.0, 0) == 1
    assert L.ming_qweight_bits(None) == 0
    assert L.ming_ctx_create(0, None, None) == 1
    # a null destroy is a no-op, and success clears the error
    assert L.ming_ctx_destroy(None) == 0
    assert L.ming_last_error() == b""


def test_context_on_a_missing_device_is_an_error_not_a_crash():
    import torch
    h = C.c_void_p()
    rc = m.lib().ming_ctx_create(64, None, C.byref(h))
    assert rc != 0 and not h.value
    assert m.lib().ming_last_error() != b""
    if not torch.cuda.is_available():
        try:
            m.Ctx(0)
        except m.MingError as e:
            assert e.code in (1, 3)
        else:
            raise AssertionError("a context without a GPU must be refused")


def test_calibration_library_exports_its_entry_point():
    """bench.py --mfma-ceiling loads libming_calib.so (built beside the
    library, outside its ABI) and calls ming_calib_mfma."""
    import os
    path = os.path.join(os.path.dirname(m.LIB_PATH), "libming_calib.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path],
                         capture_output=True, text=True, check=True).stdout
    assert " T ming_calib_mfma" in out
