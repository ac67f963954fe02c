"""The library's device code is built without packed f32 VALU ops: every HIP source, compiled for
gfx950 with the Makefile's flags, holds none in its device assembly (and a probe shows the flag is
what removes them)."""
import os
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "irontimber_amd", "csrc")
PACKED = re.compile(r"\bv_pk_(fma|mul|add)_f32\b")


def makefile_flags():
    text = open(os.path.join(CSRC, "Makefile")).read()
    m = re.search(r"^HIPFLAGS\s*:=\s*((?:.*\\\n)*.*)$", text, re.M)
    flags = m.group(1).replace("\\\n", " ").replace("$(ARCH)", "gfx950").split()
    return [f for f in flags if f not in ("-fPIC",)]


def device_asm(src, flags, out):
    cmd = ["/opt/rocm/bin/hipcc", *flags, "--cuda-device-only", "-S", src, "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, cwd=CSRC)
    return open(out).read()


def test_flag_is_in_makefile_and_effective(tmp_path):
    flags = makefile_flags()
    assert "-packed-fp32-ops" in flags
    probe = tmp_path / "probe.hip"
    probe.write_text("#include <hip/hip_runtime.h>\n"
                     "typedef float f2 __attribute__((ext_vector_type(2)));\n"
                     "__global__ void k(f2* a, const f2* b, const f2* c) { int i = threadIdx.x; a[i] = a[i] * b[i] + c[i]; }\n")
    plain = [f for f in flags if f not in ("-Xclang", "-target-feature", "-packed-fp32-ops")]
    assert PACKED.search(device_asm(str(probe), plain, str(tmp_path / "a.s")))        # the compiler would use them
    assert not PACKED.search(device_asm(str(probe), flags, str(tmp_path / "b.s")))    # the flag removes them


def test_library_device_code_has_no_packed_f32(tmp_path):
    flags = makefile_flags()
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    assert len(srcs) >= 8
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        asms = list(ex.map(lambda s: device_asm(os.path.join(CSRC, s), flags, str(tmp_path / (s + ".s"))), srcs))
    for s, a in zip(srcs, asms):
        assert not PACKED.search(a), f"{s}: packed f32 op in device code"
