"""Pins of the oracle's IQ grid-type decoders (src/gguf/dequant.rs:505-719)
beyond the reference's known answers (tests/test_oracle.py runs those from
tests/golden/gguf_kat.json):

  * the codebooks' structure (size, value set, order, no duplicates), so a
    mistyped or reordered entry fails;
  * ksigns_iq2xs against its closed form (the 128 bytes with even parity,
    in order of their low 7 bits);
  * one block per type with a single non-zero field of each kind (a grid
    index with its high bits, a sign index or byte, a sub-scale), whose
    expected lanes are written out from the format for that one case, so a
    wrong shift, mask, offset or operand fails.
"""
import numpy as np
import pytest

import oracle as orc

F16_ONE = (0x00, 0x3C)


def grid_bytes(entry, n=8):
    return [(int(entry) >> (8 * j)) & 0xFF for j in range(n)]


def signed(v):
    return v - 256 if v >= 128 else v


def block(total, d1=True):
    b = np.zeros(total, np.uint8)
    if d1:
        b[0], b[1] = F16_ONE
    return b


def sign_of(sbyte, j):
    return -1.0 if (sbyte >> j) & 1 else 1.0


@pytest.mark.parametrize("name,size,values,ordered", [
    ("iq2xxs", 256, {8, 25, 43}, True),
    ("iq2xs", 512, {8, 25, 43}, True),
    ("iq2s", 1024, {8, 25, 43}, True),
    ("iq3xxs", 256, {4, 12, 20, 28, 36, 44, 52, 62}, True),
    ("iq3s", 512, {1, 3, 5, 7, 9, 11, 13, 15}, True),
    ("iq1s", 2048, {0xFF, 0x00, 0x01}, False),
])
def test_codebook_structure(name, size, values, ordered):
    g = orc.iq_grid(name)
    nbytes = 4 if name.startswith("iq3") else 8
    assert g.size == size
    assert len(set(g.tolist())) == size, "codebook points are distinct"
    seen = set()
    for e in g.tolist():
        assert e >> (8 * nbytes) == 0
        seen.update(grid_bytes(e, nbytes))
    assert seen == values
    if ordered:
        e = [int(v) for v in g.tolist()]
        assert all(a < b for a, b in zip(e, e[1:])), "IQ2/IQ3 codebooks are stored in ascending order"
    # the entries the reference's known answers rely on (dequant.rs:884-955)
    assert int(g[0]) == {"iq2xxs": 0x0808080808080808, "iq2xs": 0x0808080808080808, "iq2s": 0x0808080808080808,
                         "iq3xxs": 0x04040404, "iq3s": 0x01010101, "iq1s": 0xFFFFFFFFFFFFFFFF}[name]


def test_ksigns_closed_form():
    k = orc.ksigns_iq2xs()
    for i, v in enumerate(k.tolist()):
        assert v & 127 == i
        assert bin(v).count("1") % 2 == 0
    assert k[:4].tolist() == [0, 129, 130, 3] and k[127] == 255


def test_iq2_xxs_fields():
    g = orc.iq_grid("iq2xxs")
    b = block(66)
    ib, l, idx, sidx, scale = 1, 2, 37, 0x55, 5
    b[2 + 8 * ib + l] = idx
    aux1 = (scale << 28) | (sidx << (7 * l))
    b[2 + 8 * ib + 4:2 + 8 * ib + 8] = np.frombuffer(np.uint32(aux1).tobytes(), np.uint8)
    y = orc.gguf_dequantize(16, b, 256)
    db = 1.0 * (0.5 + scale) * 0.25
    s = int(orc.ksigns_iq2xs()[sidx])
    want = np.ones(256, np.float32)
    want[32 * ib:32 * ib + 32] = db * 8
    for j, v in enumerate(grid_bytes(g[idx])):
        want[32 * ib + 8 * l + j] = np.float32(db * v) * sign_of(s, j)
    assert np.array_equal(y, want)


def test_iq2_xs_fields():
    g = orc.iq_grid("iq2xs")
    b = block(74)
    ib, l, idx, sidx = 2, 3, 300, 9
    q = idx | (sidx << 9)
    o = 2 + 2 * (4 * ib + l)
    b[o], b[o + 1] = q & 0xFF, q >> 8
    b[66 + ib] = 0x73  # low nibble: groups 0-1, high nibble: groups 2-3
    y = orc.gguf_dequantize(17, b, 256)
    s = int(orc.ksigns_iq2xs()[sidx])
    want = np.ones(256, np.float32)
    want[32 * ib:32 * ib + 16] = (0.5 + 3) * 0.25 * 8
    want[32 * ib + 16:32 * ib + 32] = (0.5 + 7) * 0.25 * 8
    for j, v in enumerate(grid_bytes(g[idx])):
        want[32 * ib + 8 * l + j] = np.float32((0.5 + 7) * 0.25 * v) * sign_of(s, j)
    assert np.array_equal(y, want)


def test_iq2_s_fields():
    g = orc.iq_grid("iq2s")
    b = block(82)
    ib = 5
    b[2 + 4 * ib + 1] = 0x21  # group 1: low index byte
    b[2 + 4 * ib + 3] = 0x07  # group 3
    b[66 + ib] = 0x88         # qh: bit 3 -> group 1 index bit 9, bit 7 -> group 3 index bit 9
    b[2 + 32 + 4 * ib + 1] = 0xA5  # group 1 sign byte (used as is)
    y = orc.gguf_dequantize(22, b, 256)
    want = np.ones(256, np.float32)
    for l, idx, sb in ((1, 0x221, 0xA5), (3, 0x207, 0)):
        for j, v in enumerate(grid_bytes(g[idx])):
            want[32 * ib + 8 * l + j] = np.float32(0.125 * v) * sign_of(sb, j)
    assert np.array_equal(y, want)


def test_iq3_xxs_fields():
    g = orc.iq_grid("iq3xxs")
    b = block(98)
    ib, l, i1, i2, sidx, scale = 6, 1, 17, 200, 0x33, 9
    b[2 + 8 * ib + 2 * l], b[2 + 8 * ib + 2 * l + 1] = i1, i2
    aux = (scale << 28) | (sidx << (7 * l))
    b[66 + 4 * ib:66 + 4 * ib + 4] = np.frombuffer(np.uint32(aux).tobytes(), np.uint8)
    y = orc.gguf_dequantize(18, b, 256)
    db = (0.5 + scale) * 0.5
    s = int(orc.ksigns_iq2xs()[sidx])
    want = np.ones(256, np.float32)
    want[32 * ib:32 * ib + 32] = db * 4
    vals = grid_bytes(g[i1], 4) + grid_bytes(g[i2], 4)
    for j, v in enumerate(vals):
        want[32 * ib + 8 * l + j] = np.float32(db * v) * sign_of(s, j)
    assert np.array_equal(y, want)


def test_iq3_s_fields():
    g = orc.iq_grid("iq3s")
    b = block(110)
    k, half, l = 2, 1, 2
    b[106 + k] = 0x40                 # half 1 scale nibble 4 -> 1 + 2*4 = 9, half 0 -> 1
    b[66 + 2 * k + half] = 0x30       # qh bits 4, 5: high index bit of both points of group l = 2
    q0 = 2 + 16 * k + 8 * half
    b[q0 + 2 * l], b[q0 + 2 * l + 1] = 10, 99
    b[74 + 8 * k + 4 * half + l] = 0x0F
    y = orc.gguf_dequantize(21, b, 256)
    want = np.ones(256, np.float32)
    base = 64 * k + 32 * half
    want[base:base + 32] = 9.0
    vals = grid_bytes(g[256 + 10], 4) + grid_bytes(g[256 + 99], 4)
    for j, v in enumerate(vals):
        want[base + 8 * l + j] = np.float32(9.0 * v) * sign_of(0x0F, j)
    assert np.array_equal(y, want)


def test_iq1_s_fields():
    g = orc.iq_grid("iq1s")
    b = block(50)
    ib, l = 4, 1
    h = (5 << 12) | 0x8000 | (6 << (3 * l))  # scale 2*5+1 = 11, delta -1/8, index bits 8-10 of group 1 = 6
    b[34 + 2 * ib], b[35 + 2 * ib] = h & 0xFF, h >> 8
    b[2 + 4 * ib + l] = 0x77
    y = orc.gguf_dequantize(19, b, 256)
    want = np.full(256, -0.875, np.float32)
    want[32 * ib:32 * ib + 32] = np.float32(11 * (-1 - 0.125))
    for j, v in enumerate(grid_bytes(g[0x677])):
        want[32 * ib + 8 * l + j] = np.float32(11 * (signed(v) - 0.125))
    assert np.array_equal(y, want)


def test_iq1_m_fields():
    g = orc.iq_grid("iq1s")
    b = np.zeros(56, np.uint8)
    sc = [0, (3 << 6) | (5 << 9), 0xC000, 0x3000]  # d = f16 0x3C00; block 3: sub-scales 3 and 5
    for i, w in enumerate(sc):
        b[48 + 2 * i], b[49 + 2 * i] = w & 0xFF, w >> 8
    ib = 3
    b[32 + 2 * ib] = 0xD0  # group 1: index bits 8-10 = 5, delta negative
    b[4 * ib + 1] = 0x3C
    y = orc.gguf_dequantize(29, b, 256)
    want = np.full(256, -0.875, np.float32)
    want[32 * ib:32 * ib + 8] = 7 * -0.875
    want[32 * ib + 16:32 * ib + 32] = 11 * -0.875
    for j, v in enumerate(grid_bytes(g[0x53C])):
        want[32 * ib + 8 + j] = np.float32(7 * (signed(v) - 0.125))
    assert np.array_equal(y, want)
