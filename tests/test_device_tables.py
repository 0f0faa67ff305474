"""The LDS tables of the f64 kernels (fill_tables in phz_device.h), read from
the header's text and pinned entry by entry against mpmath at 50 digits:
the sine table holds the correctly rounded cosine and sine of 2 pi k / 64
(exact zeros and ones at the quarter turns); the log table holds, for each of
its 64 intervals of z (2^-7 wide below 1, 2^-6 above, starting at the
double with high word 0x3FE62000), invc = the double nearest 1 / (the
interval's midpoint), except 1 exactly for the interval holding 1, and logc =
the double nearest -ln invc."""
import os
import re
import struct

import mpmath
import numpy as np

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "phyz_amd", "csrc", "phz_device.h")


def table(name):
    src = open(HDR).read()
    m = re.search(r"static constexpr double " + name + r"\[128\] = \{([^}]*)\}", src)
    vals = [float.fromhex(t.strip()) if "0x" in t else float(t) for t in m.group(1).split(",")]
    assert len(vals) == 128
    return np.array(vals).reshape(64, 2)


def test_sine_table_is_correctly_rounded():
    mpmath.mp.dps = 50
    tab = table("k")
    for k in range(64):
        a = 2 * mpmath.pi * k / 64
        assert tab[k, 0] == float(mpmath.cos(a)) or abs(float(mpmath.cos(a))) < 1e-40 and tab[k, 0] == 0.0
        assert tab[k, 1] == float(mpmath.sin(a)) or abs(float(mpmath.sin(a))) < 1e-40 and tab[k, 1] == 0.0
    assert tab[0].tolist() == [1.0, 0.0] and tab[16].tolist() == [0.0, 1.0]
    assert tab[32].tolist() == [-1.0, 0.0] and tab[48].tolist() == [0.0, -1.0]


def test_log_table_pins_its_intervals():
    mpmath.mp.dps = 50
    tab = table("lg")
    for i in range(64):
        lo, hi = [struct.unpack("<d", struct.pack("<Q", (0x3FE62000 + j * 2 ** 14) << 32))[0] for j in (i, i + 1)]
        invc, logc = tab[i]
        if lo <= 1.0 < hi:
            assert invc == 1.0 and logc == 0.0
        else:
            assert invc == float(1 / mpmath.mpf((lo + hi) / 2))
            assert logc == float(-mpmath.log(mpmath.mpf(invc)))
        # the reduced argument r = z invc - 1 stays within 2^-7 over the interval
        assert max(abs(lo * invc - 1), abs(hi * invc - 1)) <= 2.0 ** -7
