"""Write tests/golden/gguf_kat.json: the reference's own GGUF known-answer
vectors as data (inputs + expected outputs), taken from the literal blocks and
assertions of the reference tests:

  type_geometry_matches_llama_cpp   src/gguf/dequant.rs:725-747
  supported_and_unsupported_types   src/gguf/dequant.rs:749-766
  iq4_nl_codebook_decode            src/gguf/dequant.rs:769-780
  f32_f16_bf16_passthrough          src/gguf/dequant.rs:782-802
  q8_0_block_dequant                src/gguf/dequant.rs:805-816
  q4_0_zero_centered                src/gguf/dequant.rs:820-836
  q2_k_scale_and_unpack             src/gguf/dequant.rs:841-850
  q6_k_centered_is_zero             src/gguf/dequant.rs:854-875
  iq2_xxs_grid_scale_and_offset     src/gguf/dequant.rs:884-900
  iq2_xs_and_s_grid_zero_decode     src/gguf/dequant.rs:902-910
  iq3_xxs_and_s_grid_zero_decode    src/gguf/dequant.rs:912-920
  iq1_s_signed_grid_and_scale       src/gguf/dequant.rs:922-937
  iq1_m_packed_f16_scale            src/gguf/dequant.rs:939-955

and the two Q8 tolerance tests of src/primitives/quant.rs:91-125 (inputs and
bounds).  Nothing from the reference is imported or run; the byte strings
below are the blocks those tests build (f16 1.0 = 0x3C00, 2.0 = 0x4000,
0.5 = 0x3800; bf16 of the same values = the top half of their f32 bits).
"""
import json
import struct
from pathlib import Path

OUT = Path(__file__).resolve().with_name("gguf_kat.json")


def f16(v):
    return {1.0: 0x3C00, 2.0: 0x4000, 0.5: 0x3800, -2.5: 0xC100, 3.25: 0x4280, 0.0: 0x0000}[v]


def le16(h):
    return bytes([h & 0xFF, h >> 8])


def main():
    cases = []
    # iq4_nl_codebook_decode
    b = le16(f16(2.0)) + bytes([0x80]) + bytes(15)
    cases.append({"name": "iq4_nl_codebook_decode", "tag": 20, "n": 32, "hex": b.hex(),
                  "expect": {"0": -254.0, "16": 2.0, "1": -254.0}})
    # f32_f16_bf16_passthrough
    vals = [1.0, -2.5, 3.25, 0.0]
    cases.append({"name": "f32_passthrough", "tag": 0, "n": 4,
                  "hex": b"".join(struct.pack("<f", v) for v in vals).hex(), "expect_all": vals})
    cases.append({"name": "f16_passthrough", "tag": 1, "n": 4,
                  "hex": b"".join(le16(f16(v)) for v in vals).hex(), "expect_all": vals})
    cases.append({"name": "bf16_passthrough", "tag": 30, "n": 4,
                  "hex": b"".join(le16(struct.unpack("<I", struct.pack("<f", v))[0] >> 16) for v in vals).hex(),
                  "expect_all": vals})
    # q8_0_block_dequant: d=0.5, quants -16..15 -> (i-16)*0.5
    b = le16(f16(0.5)) + bytes(((q - 16) & 0xFF) for q in range(32))
    cases.append({"name": "q8_0_block_dequant", "tag": 8, "n": 32, "hex": b.hex(),
                  "expect_all": [(i - 16) * 0.5 for i in range(32)]})
    # q4_0_zero_centered
    b = le16(f16(1.0)) + bytes([0x88] * 16)
    cases.append({"name": "q4_0_zero_centered", "tag": 2, "n": 32, "hex": b.hex(), "expect_all": [0.0] * 32})
    b = le16(f16(1.0)) + bytes([0x8F]) + bytes([0x88] * 15)
    cases.append({"name": "q4_0_low_nibble_f", "tag": 2, "n": 32, "hex": b.hex(),
                  "expect": {"0": 7.0, "16": 0.0}})
    # q2_k_scale_and_unpack
    b = bytes([0x01] * 16) + bytes([0xFF] * 64) + le16(f16(1.0)) + le16(f16(1.0))
    cases.append({"name": "q2_k_scale_and_unpack", "tag": 10, "n": 256, "hex": b.hex(), "expect_all": [3.0] * 256})
    # q6_k_centered_is_zero
    b = bytearray(210)
    for i in range(128, 192):
        b[i] = 0xAA
    for i in range(192, 208):
        b[i] = 5
    b[208:210] = le16(f16(1.0))
    cases.append({"name": "q6_k_centered_is_zero", "tag": 14, "n": 256, "hex": bytes(b).hex(),
                  "expect_all": [0.0] * 256})

    # IQ grid types: f16 d = 1 then a zero payload (iq_block_d1, dequant.rs:877-882)
    def iq_d1(total, **patch):
        b = bytearray(le16(f16(1.0)) + bytes(total - 2))
        for k, v in patch.items():
            b[int(k[1:])] = v
        return bytes(b)

    cases.append({"name": "iq2_xxs_grid_zero", "tag": 16, "n": 256, "hex": iq_d1(66).hex(),
                  "expect_all": [1.0] * 256})
    cases.append({"name": "iq2_xxs_block0_scale3", "tag": 16, "n": 256, "hex": iq_d1(66, b9=0x30).hex(),
                  "expect_all": [7.0] * 32 + [1.0] * 224})
    cases.append({"name": "iq2_xs_grid_zero", "tag": 17, "n": 256, "hex": iq_d1(74).hex(), "expect_all": [1.0] * 256})
    cases.append({"name": "iq2_s_grid_zero", "tag": 22, "n": 256, "hex": iq_d1(82).hex(), "expect_all": [1.0] * 256})
    cases.append({"name": "iq3_xxs_grid_zero", "tag": 18, "n": 256, "hex": iq_d1(98).hex(),
                  "expect_all": [1.0] * 256})
    cases.append({"name": "iq3_s_grid_zero", "tag": 21, "n": 256, "hex": iq_d1(110).hex(), "expect_all": [1.0] * 256})
    cases.append({"name": "iq1_s_signed_grid", "tag": 19, "n": 256, "hex": iq_d1(50).hex(),
                  "expect_all": [-0.875] * 256})
    cases.append({"name": "iq1_s_block0_scale3", "tag": 19, "n": 256, "hex": iq_d1(50, b35=0x10).hex(),
                  "expect_all": [-2.625] * 32 + [-0.875] * 224})
    b = bytearray(56)
    b[53] = 0xC0  # sc2 = 0xC000
    b[55] = 0x30  # sc3 = 0x3000 -> d = f16 0x3C00 = 1.0
    cases.append({"name": "iq1_m_packed_f16_scale", "tag": 29, "n": 256, "hex": bytes(b).hex(),
                  "expect_all": [-0.875] * 256})
    cases.append({"name": "iq1_m_zero_scale", "tag": 29, "n": 256, "hex": bytes(56).hex(), "expect_all": [0.0] * 256})

    geometry = {  # dequant.rs:727-746 (tag: [elems, bytes])
        "2": [32, 18], "3": [32, 20], "6": [32, 22], "7": [32, 24], "8": [32, 34], "10": [256, 84],
        "11": [256, 110], "12": [256, 144], "13": [256, 176], "14": [256, 210], "20": [32, 18],
        "23": [256, 136], "16": [256, 66], "17": [256, 74], "22": [256, 82], "18": [256, 98],
        "21": [256, 110], "19": [256, 50], "29": [256, 56],
    }
    supported = [20, 23, 16, 17, 18, 19, 21, 22, 29]  # dequant.rs:751-760
    unsupported = [9, 15]                             # dequant.rs:763-765
    byte_len = [[16, 256, 66]]                        # dequant.rs:761

    # quant.rs:91-107 and :111-125 inputs (f32) and their bounds
    affine = {
        "roundtrip_q8": {"shape": [2, 64], "w": [i / 128.0 - 0.5 for i in range(128)], "bits": 8,
                         "group_size": 64, "max_abs_err": 0.01},
        "matmul_q8": {"shape": [4, 64], "w": [((i * 7 % 13) / 13.0) - 0.5 for i in range(256)],
                      "x": [i / 64.0 - 0.5 for i in range(64)], "bits": 8, "group_size": 64,
                      "max_abs_err": 0.05},
    }
    OUT.write_text(json.dumps({"cases": cases, "geometry": geometry, "supported_tags": supported,
                               "unsupported_tags": unsupported, "byte_len": byte_len, "affine": affine},
                              indent=1))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
