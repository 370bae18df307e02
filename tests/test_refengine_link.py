# SPDX-License-Identifier: MPL-2.0
"""CPU checks of the drop-in boundary against the reference tree (skipped
where the reference checkout is absent):

- the reference's C engine, compiled from its sources with its own CFLAGS
  (oracle/Makefile `refengine`), links against libbaremetal_hip.so with no
  undefined symbol (the link uses -Wl,--no-undefined) and needs no Metal
  framework;
- the fields of the backend context the reference's engine reads
  (`supports_bf16`, api.c:30; `library`, cli.c:98) sit at the same offsets
  in include/backend_hip_device.h as in the reference's
  src/backend/metal/device.h, so objects compiled against either header
  read the HIP context correctly."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
REFENGINE = os.path.join(ROOT, "oracle", "_ref", "refengine")

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REF, "src", "baremetal", "scheduler.c")),
                                reason="reference tree absent")


def test_reference_engine_links_against_the_library():
    if not os.path.exists(os.path.join(ROOT, "bare.metal_amd", "libbaremetal_hip.so")):
        pytest.skip("library not built")
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "refengine"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    dyn = subprocess.run(["readelf", "-d", REFENGINE], capture_output=True, text=True, check=True).stdout
    needed = [ln.split("[")[1].rstrip("]") for ln in dyn.splitlines() if "(NEEDED)" in ln]
    assert "libbaremetal_hip.so" in needed, needed
    assert not any("Metal" in n or "Foundation" in n for n in needed), needed


def _offsets(tmp_path, header_dir, header, tag):
    src = tmp_path / f"off_{tag}.c"
    src.write_text(f'#include <stddef.h>\n#include <stdint.h>\n#include <stdio.h>\n#include "{header}"\n'
                   "int main(void) { printf(\"%zu %zu %zu %zu\\n\", offsetof(struct backend_ctx_s, device), "
                   "offsetof(struct backend_ctx_s, queue), offsetof(struct backend_ctx_s, library), "
                   "offsetof(struct backend_ctx_s, supports_bf16)); return 0; }\n")
    exe = tmp_path / f"off_{tag}"
    subprocess.run(["gcc", "-std=c11", "-I", header_dir, str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()


def test_device_header_fields_match_reference(tmp_path):
    ref = _offsets(tmp_path, os.path.join(REF, "src"), "backend/metal/device.h", "ref")
    ours = _offsets(tmp_path, os.path.join(ROOT, "include"), "backend_hip_device.h", "hip")
    assert ours == ref, (ours, ref)
