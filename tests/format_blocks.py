"""Packed block formats for the tests: ids, block geometry and builders of
valid packed blocks (ggml block layouts, restated in oracle/formats.c)."""
import numpy as np

Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 1, 2, 3, 4, 5, 6, 7, 8, 9, 10
IQ4_NL, IQ4_XS = 16, 17
LEGACY = [Q8_0, Q4_0, Q4_1, Q5_0, Q5_1]
KQUANT = [Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]
IQ = [IQ4_NL, IQ4_XS]
ALL = LEGACY + KQUANT + IQ
# ggml's IQ4_NL / IQ4_XS code book (kvalues_iq4nl)
IQ4NL_TABLE = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
NAMES = {Q8_0: "Q8_0", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", Q2_K: "Q2_K",
         Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ4_NL: "IQ4_NL", IQ4_XS: "IQ4_XS"}
# elements and bytes per block
GEOM = {Q8_0: (32, 34), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24),
        Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
        IQ4_NL: (32, 18), IQ4_XS: (256, 136)}


def f16_bytes(v):
    return np.array([v], np.float16).view(np.uint8)


def random_blocks(fmt, rows, cols, rng, scale=None):
    """Packed blocks of random codes and random finite fp16 scales, sized so a
    row of N(0,1) inputs gives outputs of order one."""
    qk, bb = GEOM[fmt]
    nb = rows * cols // qk
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    s = scale if scale is not None else 1.0 / np.sqrt(cols)
    d = (rng.uniform(0.5, 1.5, nb) * s / (8 if fmt != Q8_0 else 64)).astype(np.float16)
    m = (rng.uniform(-1.0, 1.0, nb) * s).astype(np.float16)
    if fmt in (Q8_0, Q4_0, Q5_0):
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    elif fmt in (Q4_1, Q5_1):
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
    elif fmt in (Q4_K, Q5_K):
        dk = (d.astype(np.float32) / 32).astype(np.float16)  # 6-bit sub-block scales
        raw[:, 0:2] = dk.view(np.uint8).reshape(nb, 2)
        mk = (np.abs(m.astype(np.float32)) / 32).astype(np.float16)
        raw[:, 2:4] = mk.view(np.uint8).reshape(nb, 2)
    elif fmt == Q2_K:  # 4-bit sub-block scales and mins, f16 d, dmin at the end
        raw[:, 80:82] = (d.astype(np.float32) / 8).astype(np.float16).view(np.uint8).reshape(nb, 2)
        raw[:, 82:84] = (np.abs(m.astype(np.float32)) / 16).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif fmt == Q3_K:  # signed 6-bit scales (-32..31), f16 d at the end
        raw[:, 108:110] = (d.astype(np.float32) / 16).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif fmt == IQ4_NL:  # codes up to 127 in magnitude
        raw[:, 0:2] = (d.astype(np.float32) / 16).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif fmt == IQ4_XS:  # and 6-bit scales (-32..31)
        raw[:, 0:2] = (d.astype(np.float32) / 256).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif fmt == Q6_K:
        dk = (d.astype(np.float32) / 64).astype(np.float16)  # int8 sub-block scales
        raw[:, 208:210] = dk.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)
