"""CPU checks of constant tables compiled into the device code."""
import os
import re
import struct
from decimal import Decimal, getcontext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exp2_table_regenerated_from_its_definition():
    # kExp2Tab[i] = asuint64(double(2^(i/32))) - (i << 47) (common.h, dev_expf)
    text = open(os.path.join(ROOT, "prana_amd", "csrc", "common.h")).read()
    body = text[text.index("kExp2Tab[32] = {"):]
    body = body[:body.index("};")]
    tab = [int(h, 16) for h in re.findall(r"0x([0-9a-f]{16})ull", body)]
    assert len(tab) == 32
    getcontext().prec = 60
    for i in range(32):
        v = float(Decimal(2) ** (Decimal(i) / Decimal(32)))  # correctly rounded to double
        bits = struct.unpack("<Q", struct.pack("<d", v))[0]
        assert (bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF == tab[i], i
