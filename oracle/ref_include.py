"""Test infrastructure: a copy of the reference's engine/include with the HipOptions /
make_hip_backend block that INTEGRATION.md adds to relay/backend.h (next to CudaOptions,
backend.h:84-98), for building this backend against relay's own headers.

    python3 oracle/ref_include.py REF_INCLUDE INTEGRATION_MD OUT_DIR
"""
import os
import re
import shutil
import sys


def main(ref_include: str, integration_md: str, out: str) -> None:
    text = open(integration_md).read()
    m = re.search(r"```cpp\n(#ifdef RELAY_HIP\nstruct HipOptions.*?#endif)\n```", text, re.S)
    if not m:
        raise SystemExit("INTEGRATION.md has no HipOptions block")
    if os.path.isdir(out):
        shutil.rmtree(out)
    shutil.copytree(ref_include, out)
    path = os.path.join(out, "relay", "backend.h")
    header = open(path).read()
    anchor = "}  // namespace relay"
    i = header.rindex(anchor)
    open(path, "w").write(header[:i] + m.group(1) + "\n" + header[i:])


if __name__ == "__main__":
    main(*sys.argv[1:4])
