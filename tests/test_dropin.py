"""The drop-in boundary, checked against relay's own headers: hip_backend.cpp and capi.cpp
compile against the reference's engine/include/relay/*.h (with the HipOptions /
make_hip_backend declarations INTEGRATION.md adds next to CudaOptions,
engine/include/relay/backend.h:84-98), not only against this build's restatement of them
(relay_amd/csrc/host/relay/*.h). A restated header that drifts from relay's, or backend
code that uses something relay's headers do not declare, fails here. CPU only (g++
-fsyntax-only); skipped where the reference tree is absent (the GPU box)."""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/engine/include"
HOST = os.path.join(REPO, "relay_amd", "csrc", "host")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference tree not present")


def _integration_block():
    """The HipOptions block as INTEGRATION.md prints it (so the document and this test agree)."""
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    m = re.search(r"```cpp\n(#ifdef RELAY_HIP\nstruct HipOptions.*?#endif)\n```", text, re.S)
    assert m, "INTEGRATION.md no longer shows the HipOptions block"
    return m.group(1)


def _patched_include(tmp):
    inc = os.path.join(tmp, "include")
    shutil.copytree(REF_INCLUDE, inc)
    path = os.path.join(inc, "relay", "backend.h")
    text = open(path).read()
    anchor = "}  // namespace relay"
    assert text.rstrip().endswith(anchor) or anchor in text
    i = text.rindex(anchor)
    open(path, "w").write(text[:i] + _integration_block() + "\n" + text[i:])
    return inc


def _compile(src, includes, tmp):
    # The sources are copied out of relay_amd/csrc/host so that their own directory (with the
    # restated relay/*.h) is not on the include path.
    work = os.path.join(tmp, "src")
    os.makedirs(work, exist_ok=True)
    for h in ("host_common.h", "lt_gemm.h"):
        shutil.copy(os.path.join(HOST, h), work)
    dst = os.path.join(work, os.path.basename(src))
    shutil.copy(src, dst)
    cmd = ["g++", "-std=c++20", "-fsyntax-only", "-DRELAY_HIP=1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           *[f"-I{i}" for i in includes], f"-I{os.path.join(REPO, 'include')}", dst]
    return subprocess.run(cmd, capture_output=True, text=True)


def test_integration_block_matches_the_restated_header():
    block = _integration_block()
    restated = open(os.path.join(HOST, "relay", "backend.h")).read()
    for decl in ("struct HipOptions", "bool reference_attention = false;", "bool int8_weights = false;",
                 "static HipOptions from_env();", "std::unique_ptr<Backend> make_hip_backend("):
        assert decl in block and decl in restated, decl


@pytest.mark.parametrize("name", ["hip_backend.cpp", "capi.cpp"])
def test_backend_compiles_against_relays_headers(tmp_path, name):
    inc = _patched_include(str(tmp_path))
    r = _compile(os.path.join(HOST, name), [inc], str(tmp_path))
    assert r.returncode == 0, r.stderr[-4000:]


def test_check_catches_a_drifted_header(tmp_path):
    """The check has teeth: a relay header without a member the backend uses fails."""
    inc = _patched_include(str(tmp_path))
    path = os.path.join(inc, "relay", "backend.h")
    text = open(path).read()
    assert "all_logits" in text
    open(path, "w").write(text.replace("all_logits", "all_logits_renamed"))
    r = _compile(os.path.join(HOST, "hip_backend.cpp"), [inc], str(tmp_path))
    assert r.returncode != 0
