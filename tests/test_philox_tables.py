"""The Box-Muller lookup tables of the Philox kernel (ltx-nv_amd/csrc/
philox_tables.h): the committed header is what its generator writes, and each
entry is the fp64 value it claims (the libm value of the same expression
within a few ulps, exact zeros and ones where the angle has them)."""

import math
import pathlib
import re
import subprocess
import sys

CSRC = pathlib.Path(__file__).resolve().parents[1] / "ltx-nv_amd" / "csrc"


def _tables():
    text = (CSRC / "philox_tables.h").read_text()
    hi = int(re.search(r"kLogHi = (\d+);", text).group(1))
    log_body = text.split("kLogTab[128][2] = {")[1].split("};")[0]
    sc_body = text.split("kSinCosTab[64][2] = {")[1].split("};")[0]

    def rows(body):
        out = []
        for a, b in re.findall(r"\{([^,{}]+), ([^,{}]+)\}", body):
            out.append(tuple(float.fromhex(v) if "x" in v else float(v) for v in (a.strip(), b.strip())))
        return out

    return hi, rows(log_body), rows(sc_body)


def test_header_is_the_generators_output():
    out = subprocess.run([sys.executable, str(CSRC / "gen_philox_tables.py")], capture_output=True, text=True,
                         check=True).stdout
    assert out == (CSRC / "philox_tables.h").read_text()


def test_log_table_entries():
    hi, log, _ = _tables()
    assert len(log) == 128 and 0 < hi < 128
    for i, (inv_c, t) in enumerate(log):
        c = 1 + (i + (1 if i >= hi else 0)) / 128
        assert abs(inv_c * c - 1) <= 2 ** -52, i
        want = math.log(c) - (math.log(2) if i >= hi else 0.0)  # two libm roundings and a subtraction
        assert abs(t - want) <= 3e-16, (i, t, want)
    assert log[0] == (1.0, 0.0)  # u = 1 gives exactly ln u = 0
    assert log[127][1] == 0.0 and log[127][0] == 0.5  # the top bin centred on 2: no cancellation as u -> 1


def test_sincos_table_entries():
    _, _, sc = _tables()
    assert len(sc) == 64
    for k, (s, c) in enumerate(sc):
        a = k * math.pi / 32  # rounded angle: libm's values carry its error (up to ~5e-16 here)
        assert abs(s - math.sin(a)) <= 1e-15 and abs(c - math.cos(a)) <= 1e-15, k
        assert abs(s * s + c * c - 1) <= 4e-16
    assert sc[0] == (0.0, 1.0) and sc[16] == (1.0, 0.0) and sc[32] == (0.0, -1.0) and sc[48] == (-1.0, 0.0)
