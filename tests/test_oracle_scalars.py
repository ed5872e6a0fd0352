"""Pin the oracle's scalar decoders against independent definitions.

mo_f16_to_f32 (engine/mten.h:49-57) against numpy's IEEE binary16 over all
65536 encodings; mo_fp4_value (engine/mten.h:44-47) against the OCP MX E2M1
value table; both against the compiled reference where it was built.
"""
import numpy as np
import pytest

from oracle import pyoracle as po


def test_f16_exhaustive_vs_numpy():
    lib = po.oracle()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.mo_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert (got[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all()
    # NaN payloads survive as the reference's bit construction does
    assert (got[nan].view(np.uint32) & 0x7F800000 == 0x7F800000).all()


@pytest.mark.skipif(not po.have_ref(), reason="reference engine not built here")
def test_f16_exhaustive_vs_reference():
    r = po.ref()
    lib = po.oracle()
    for b in range(65536):
        a = np.float32(lib.mo_f16_to_f32(b)).view(np.uint32)
        c = np.float32(r.ref_f16(b)).view(np.uint32)
        assert a == c, hex(b)


# OCP Microscaling spec, E2M1: magnitudes for codes 0..7; bit 3 is the sign.
E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_fp4_table():
    for code in range(16):
        v = po.fp4_value(code)
        mag = E2M1[code & 7]
        want = -mag if code & 8 else mag
        assert v == want
        assert np.signbit(np.float32(v)) == bool(code & 8), code   # code 8 is -0.0


def test_fp4_brute_force_format():
    # every E2M1 code is (-1)^s * 2^(e-1) * (1 + m/2) for e > 0, (-1)^s * m/2 for e == 0
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        want = (m / 2.0) if e == 0 else 2.0 ** (e - 1) * (1 + m / 2.0)
        assert abs(po.fp4_value(code)) == want
        assert np.signbit(np.float32(po.fp4_value(code))) == bool(s)
