"""The device rot_of's float sin/cos method (getting-over-it-rl_amd/csrc/b2_math.hpp, constants in b2_sincos_table.h)
restated on the CPU (tests/sincos_check.c) against the oracle's definition (float)sin((double)x) and
(float)cos((double)x) of the C library (the trig patch's definition, scripts/patches/box2d-2.3.1-trig.patch:17-23).

The full check covers every float with |x| < 2^20 (2 x 1.23e9 inputs, about 15 s on 8 cores); set
GOI_SINCOS_EXHAUSTIVE=1 to run it, otherwise every 5th bit pattern of the range plus dense ranges. The device side is
checked against the oracle on the GPU by test_gpu_parity.py::test_sincos_correctly_rounded."""
import os
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
TOP = 0x49800000  # 2^20


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    d = tmp_path_factory.mktemp("sincos")
    exes = {}
    for name, extra in (("table", []), ("planted", ["-DPLANT_FACTORED"])):
        exe = d / name
        subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", *extra, "-o", str(exe),
                        str(HERE / "sincos_check.c"), "-lm"], check=True)
        exes[name] = exe
    return exes


def _run(exe, lo, hi, stride=1):
    r = subprocess.run([str(exe), hex(lo), hex(hi), str(stride)], capture_output=True, text=True)
    last = r.stdout.strip().splitlines()[-1]
    assert last.startswith("checked "), r.stdout
    n, bad = int(last.split()[1]), int(last.split()[3])
    return n, bad, r.stdout


# sin(9830.4f) (0x4619999a) sits within about 2^-52 relative of a float rounding boundary: the factored addition
# formulas St cos r + Ct sin r round it the wrong way; the table value added last (St + (St (cos r - 1) + Ct sin r))
# does not.
HARD = 0x4619999a


@pytest.mark.parametrize("sign", [0, 0x80000000])
def test_table_sincos_matches_libm(checker, sign):
    if os.environ.get("GOI_SINCOS_EXHAUSTIVE") == "1":
        n, bad, out = _run(checker["table"], sign, sign + TOP)
        assert n == TOP and bad == 0, out
        return
    n, bad, out = _run(checker["table"], sign, sign + TOP, 5)
    assert n == (TOP + 4) // 5 and bad == 0, out
    for lo, hi in ((0x3f000000, 0x40000000), (HARD - (1 << 20), HARD + (1 << 20)), (0, 1 << 20)):
        n, bad, out = _run(checker["table"], sign + lo, sign + hi)
        assert n == hi - lo and bad == 0, out


def test_check_catches_factored_formulas(checker):
    n, bad, out = _run(checker["planted"], HARD - (1 << 20), HARD + (1 << 20))
    assert bad >= 1 and "x=0x1.33333" in out, out
