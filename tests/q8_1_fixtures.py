"""Fixture data of the reference's Q8_1 tests, regenerated from the formulas
those tests state (crates/nvidia/tests/q4_q8_1.rs:7-93 and
q6_q8_1.rs:13-103): 5 rows x 768 inputs of Q4_K / Q6_K blocks with fixed
scale tables and dyadic d, exact (dyadic) and lossy activation vectors, and
the 5-block packing fixture of crates/nvidia/tests/cuda_activation.rs:14-40
with its expected words."""
import numpy as np

INPUTS = 768
ROWS = 5
D_BITS = (0x2C00, 0x3000, 0x3400)


def half_value(bits: int) -> float:
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def q4k_fixture():
    """[ROWS * 3] blocks: (encoded bytes, quants[256], scales[8], minima[8], d, dmin)."""
    scales = [1, 17, 33, 63, 32, 47, 62, 48]
    minima = [63, 32, 17, 1, 47, 48, 33, 62]
    out = []
    for seed in range(ROWS * (INPUTS // 256)):
        d_bits = D_BITS[seed % 3]
        m_bits = (0x2800, 0x2C00, 0x3000)[seed % 3]
        enc = np.zeros(144, np.uint8)
        enc[0:2] = np.array([d_bits], "<u2").view(np.uint8)
        enc[2:4] = np.array([m_bits], "<u2").view(np.uint8)
        for g in range(4):
            enc[4 + g] = scales[g] | ((scales[g + 4] >> 4) << 6)
            enc[8 + g] = minima[g] | ((minima[g + 4] >> 4) << 6)
            enc[12 + g] = (scales[g + 4] & 15) | ((minima[g + 4] & 15) << 4)
        quants = np.array([(i * 7 + seed * 3 + i // 32) % 16 for i in range(256)], np.uint8)
        for g in range(8):
            for i in range(32):
                enc[16 + (g // 2) * 32 + i] |= quants[g * 32 + i] << ((g % 2) * 4)
        out.append((enc, quants, scales, minima, half_value(d_bits), half_value(m_bits)))
    return out


def q6k_fixture():
    """[ROWS * 3] blocks: (encoded bytes, quants[256] signed, scales[16], d)."""
    scales = [3, -5, 11, -13, 19, -23, 29, -31, 7, -9, 15, -17, 21, -25, 27, -2]
    out = []
    for seed in range(ROWS * (INPUTS // 256)):
        d_bits = D_BITS[seed % 3]
        enc = np.zeros(210, np.uint8)
        quants = np.array([(i * 7 + seed * 3 + i // 32) % 64 - 32 for i in range(256)], np.int16)
        for g in range(8):
            low_base = (g // 4) * 64 + (g % 2) * 32
            low_shift = 0 if g % 4 < 2 else 4
            high_base = 128 + (g // 4) * 32
            high_shift = (g % 4) * 2
            for i in range(32):
                u = int(quants[g * 32 + i]) + 32
                enc[low_base + i] |= (u & 15) << low_shift
                enc[high_base + i] |= ((u >> 4) & 3) << high_shift
        enc[192:208] = np.array(scales, np.int8).view(np.uint8)
        enc[208:210] = np.array([d_bits], "<u2").view(np.uint8)
        out.append((enc, quants, scales, half_value(d_bits)))
    return out


def activations(exact: bool) -> np.ndarray:
    vals = []
    for i in range(INPUTS):
        if exact:
            integer = 127 if i % 32 == 0 else (-127 if i % 32 == 1 else (i * 7) % 17 - 8)
            vals.append(np.float32(integer) * np.float32((0.25, 0.125, 0.0625)[(i // 32) % 3]))
        else:
            vals.append(np.float32((i * 17 + 3) % 101 - 50) * np.float32(0.0137))
    return np.array(vals, np.float32)


def encoded_rows(blocks) -> np.ndarray:
    """Blocks of the fixture as one [ROWS, 3 * block bytes] encoding (row-major)."""
    return np.concatenate([b[0] for b in blocks])


def pack_kat_input() -> np.ndarray:
    """cuda_activation.rs:14-27: five blocks, the first all zero."""
    v = np.zeros(160, np.float32)
    for block in range(1, 5):
        s = (0.0, 1.0, 0.5, 2.0, 0.25)[block]
        base = block * 32
        for off, val in ((0, 127.0), (1, -127.0), (2, 0.5), (3, -0.5), (4, 1.5), (5, -1.5), (31, 2.0)):
            v[base + off] = np.float32(val) * np.float32(s)
    return v


PACK_KAT_HEADERS = (0x4000_3C00, 0x3C00_3800, 0x4400_4000, 0x3800_3400)


def pack_kat_words() -> np.ndarray:
    """The words cuda_activation.rs:31-39 asserts for pack_kat_input()."""
    words = np.zeros(45, np.uint32)
    for block, header in enumerate(PACK_KAT_HEADERS):
        w = words[(block + 1) * 9:(block + 2) * 9]
        w[0] = header
        w[1] = 0xFF01_817F
        w[2] = 0x0000_FE02
        w[8] = 0x0200_0000
    return words
