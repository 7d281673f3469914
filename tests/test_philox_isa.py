"""The Philox kernel's instruction counts that bench.py's ALU roofline uses,
recounted from a fresh gfx950 device-assembly build of csrc/philox.hip (the
build flags of build_lib.py): VALU instructions and fp64 flops (FMA = 2) per
hardware thread of philox_normal_vec<float>, which draws 16 normals."""
import collections
import pathlib
import re
import shutil
import subprocess
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("hipcc") is None and not pathlib.Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_philox_instruction_counts_match_bench(tmp_path):
    sys.path.insert(0, str(REPO / "ltx-nv_amd"))
    import build_lib

    import bench

    out = tmp_path / "philox.s"
    cmd = [build_lib.hipcc(), *build_lib.FLAGS, "--cuda-device-only", "-S",
           str(REPO / "ltx-nv_amd" / "csrc" / "philox.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    asm = out.read_text()
    names = [m for m in re.findall(r"^(_Z\S*philox_normal_vec\S*):", asm, re.M) if "IfE" in m]
    assert len(names) == 1, names
    a = asm.index(names[0] + ":")
    body = asm[a:asm.index("s_endpgm", a)]
    ops = collections.Counter(t.split()[0] for t in (ln.strip() for ln in body.splitlines())
                              if t.startswith("v_"))
    valu = sum(ops.values())
    fma = sum(n for op, n in ops.items() if op.startswith(("v_fma_f64", "v_fmac_f64")))
    flops = 2 * fma + sum(n for op, n in ops.items() if op.startswith(("v_mul_f64", "v_add_f64")))
    assert (valu, flops) == (bench.PHILOX_VALU, bench.PHILOX_FP64_FLOPS)
