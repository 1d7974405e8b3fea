"""The oracle's element codecs against the compiled reference codecs.

Golden data (tests/golden, written by gen_golden.py from the reference's own
float_codecs.cpp compiled in this repository's oracle/_ref) pins:
  * the full decode tables (E4M3 256, E5M2 256, FP4 16 entries, f32 bits);
  * ~6.5k edge-case encodes;
  * digests of the encoder over all 2^32 f32 inputs.
Hand-derived special cases from the reference rules (float_codecs.cpp:57-200)
are checked as well, so a transcription slip fails two independent checks.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")
DT = {"e4m3": 4, "e5m2": 5, "fp4": 16}


def bits(x):
    return int(np.array(x, dtype=np.float32).view(np.uint32))


@pytest.mark.parametrize("name", list(DT))
def test_decode_table_matches_reference(oracle, name):
    tab = np.load(os.path.join(GOLD, "codec_tables.npz"))[name]
    n = 16 if name == "fp4" else 256
    mine = np.array([oracle.decode(DT[name], c) for c in range(n)], np.float32).view(np.uint32)
    assert np.array_equal(mine, tab)


@pytest.mark.parametrize("name", list(DT))
def test_encode_samples_match_reference(oracle, name):
    s = np.load(os.path.join(GOLD, "codec_samples.npz"))
    xs = s["bits"].view(np.float32)
    assert np.array_equal(oracle.encode_array(DT[name], xs), s[name])


@pytest.mark.parametrize("name", list(DT))
def test_encode_all_2e32_inputs_match_reference(oracle, name):
    gold = np.load(os.path.join(GOLD, "codec_sweep.npz"))[name]
    assert np.array_equal(oracle.sweep(DT[name]), gold)


def test_sweep_digest_detects_one_wrong_code(oracle):
    # The digest pair changes when a single code in a chunk changes.
    gold = np.load(os.path.join(GOLD, "codec_sweep.npz"))["e4m3"]
    d = oracle.sweep(4, first=0x3F8, n=1)[0].copy()
    assert np.array_equal(d, gold[0x3F8])
    d[0] += 1
    d[1] += 7
    assert not np.array_equal(d, gold[0x3F8])


def test_e4m3_rules(oracle):
    e = lambda x: oracle.encode(4, x)
    assert e(0.0) == 0 and e(-0.0) == 0 and e(float("nan")) == 0
    assert e(1.0) == 0x38 and e(-1.0) == 0xB8
    assert e(240.0) == 0x77
    assert e(247.9) == 0x77
    assert e(248.0) == 0x7E and e(300.0) == 0x7E and e(448.0) == 0x7E
    assert e(float("inf")) == 0x7E and e(float("-inf")) == 0xFE
    # half-away rounding on one guard bit: 1 + 1/16 -> 1 + 1/8
    assert e(1.0 + 2 ** -4) == 0x39
    assert e(np.nextafter(np.float32(1.0 + 2 ** -4), np.float32(0))) == 0x38
    # subnormal range is truncated: 2^-7 (E = 0) -> mantissa 4
    assert e(2.0 ** -7) == 0x04
    assert e(2.0 ** -9) == 0x01
    assert e(2.0 ** -10) == 0x00
    assert e(-(2.0 ** -12)) == 0x80


def test_e4m3_decode_rules(oracle):
    d = lambda c: oracle.decode(4, c)
    for m in range(8):
        assert d(m) == 0.0 and np.signbit(np.float32(d(0x80 | m)))
    assert d(0x7F) == 448.0 and d(0xFF) == -448.0
    assert d(0x7E) == 448.0 and d(0x77) == 240.0 and d(0x08) == 2.0 ** -6


def test_e5m2_rules(oracle):
    e = lambda x: oracle.encode(5, x)
    assert e(float("nan")) == 0x7E
    assert e(-0.0) == 0x80 and e(0.0) == 0x00
    assert e(float("inf")) == 0x7C and e(float("-inf")) == 0xFC
    assert e(57344.0) == 0x7B and e(61439.0) == 0x7B and e(61440.0) == 0x7C
    assert e(2.0 ** -14) == 0x04 and e(2.0 ** -15) == 0x00
    d = lambda c: oracle.decode(5, c)
    assert d(0x01) == 0.0 and d(0x7C) == float("inf") and np.isnan(d(0x7D))
    assert bits(d(0xFD)) == 0xFFC00000


def test_fp4_rules(oracle):
    e = lambda x: oracle.encode(16, x)
    # ties go to the lower index (smaller magnitude)
    assert e(0.25) == 0 and e(0.75) == 1 and e(2.5) == 4 and e(5.0) == 6
    assert e(-0.75) == 9 and e(-5.0) == 14
    assert e(-0.1) == 0  # code 8 (-0) is never produced
    assert e(7.0) == 7 and e(-100.0) == 15
    assert e(float("nan")) == 0 and e(float("inf")) == 0 and e(float("-inf")) == 0
    # f32 cancellation for huge inputs collapses the errors: lowest index wins
    assert e(2.0 ** 30) == 0
    for c in range(16):
        v = oracle.decode(16, c)
        assert oracle.decode(16, e(v)) == v


@pytest.mark.parametrize("name", ["e4m3", "e5m2"])
def test_decode_encode_roundtrip_on_code_values(oracle, name):
    dt = DT[name]
    for c in range(256):
        v = oracle.decode(dt, c)
        if np.isnan(v):
            continue
        if dt == 4 and 240.0 < abs(v) < 448.0:
            # codes 0x78-0x7D are never produced: |x| >= 248 encodes to 448
            assert oracle.encode(dt, v) in (0x7E, 0xFE)
            continue
        back = oracle.encode(dt, v)
        assert oracle.decode(dt, back) == v or (v == 0.0)
