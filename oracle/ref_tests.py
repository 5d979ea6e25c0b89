"""Test infrastructure: relay's own test programs, set up to run on the HIP backend.

Writes OUT_DIR/check.h -- the reference's tests/check.h with the RELAY_TEST_BACKEND=hip branch
that INTEGRATION.md adds to check::make_backend (tests/check.h:62-73) -- and copies the named
test sources next to it, so that their `#include "check.h"` finds the patched harness. The
output directory is build output (oracle/_ref/, git-ignored); nothing here is committed.

    python3 oracle/ref_tests.py REF_TESTS_DIR INTEGRATION_MD OUT_DIR test_transfer.cpp ...
"""
import os
import re
import shutil
import sys

ANCHOR = "  return relay::make_cpu_backend(w, blocks, block_size);"


def main(ref_tests: str, integration_md: str, out: str, *sources: str) -> None:
    text = open(integration_md).read()
    m = re.search(r"```cpp\n(  if \(test_backend\(\) == \"hip\"\) \{\n.*?\n  \})\n```", text, re.S)
    if not m:
        raise SystemExit("INTEGRATION.md has no RELAY_TEST_BACKEND=hip block")
    check = open(os.path.join(ref_tests, "check.h")).read()
    if check.count(ANCHOR) != 1:
        raise SystemExit("check.h: make_backend's final return not found")
    os.makedirs(out, exist_ok=True)
    patched = check.replace(ANCHOR, m.group(1) + "\n" + ANCHOR)
    with open(os.path.join(out, "check.h"), "w") as f:
        f.write(patched)
    for s in sources:
        shutil.copyfile(os.path.join(ref_tests, s), os.path.join(out, s))


if __name__ == "__main__":
    main(*sys.argv[1:])
