"""The reference-side binding shown in INTEGRATION.md (the C++ stub class a
maintainer would add to ming-dit.cc) compiles against include/ming_dit_amd.h:
a changed signature in the header breaks this test instead of the document
silently drifting from the ABI. Syntax only (g++ -fsyntax-only); nothing runs."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_integration_stub_compiles_against_the_header(tmp_path):
    if not shutil.which("g++") or not os.path.isdir("/opt/rocm/include/hip"):
        pytest.skip("needs g++ and the HIP headers")
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```cpp\n(.*?)```", text, re.S)
    assert blocks, "INTEGRATION.md holds no C++ stub"
    # the first block is the stub class itself; the later ones are excerpts
    # that live inside the reference's own member functions
    blocks = blocks[:1]
    src = tmp_path / "stub.cc"
    src.write_text("#include <hip/hip_runtime_api.h>\n#include <cstdint>\n#include <string>\n"
                   "#include <vector>\n" + "\n".join(blocks))
    r = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__",
                        "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
