#!/usr/bin/env python3
"""Writes the i-quant codebooks of the GEMV / dequantizer formats IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S as
compact code words (qwengine_amd/csrc/iq_grids.inc) and the SHA-256 of every expanded byte table
(tests/golden/iq_grids_sha256.json).

The codebooks are format data: a GGUF weight decodes to the values of ggml's grid tables, so the library must
reproduce them exactly.  The source is the reference's copy of those tables (src/quant/iq_tables.inc:38-370,
itself taken from ggml-common.h).  Every grid byte of a table is one of a few levels -- IQ2: 8, 25, 43; IQ3_XXS:
4, 12, 20, 28, 36, 44, 52, 62; IQ3_S: 1, 3, ..., 15 -- so an entry is written as the level indices of its bytes
(2 bits per byte for IQ2, 3 bits for IQ3), byte j at bits [b j, b j + b).  The checksums let the CPU tests pin the
expansion of these code words against the reference's bytes without the reference present.

Run in the build container (where /root/reference exists): python tests/golden/make_iq_grids.py
"""
import hashlib
import json
import os
import re

REF = "/root/reference/src/quant/iq_tables.inc"
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT_INC = os.path.join(ROOT, "qwengine_amd", "csrc", "iq_grids.inc")
OUT_SHA = os.path.join(HERE, "iq_grids_sha256.json")

# name in the reference, our name, bytes per entry, levels, bits per level index
TABLES = [
    ("iq2xxs_grid", "IQ2XXS", 8, [8, 25, 43], 2),
    ("iq2xs_grid", "IQ2XS", 8, [8, 25, 43], 2),
    ("iq2s_grid", "IQ2S", 8, [8, 25, 43], 2),
    ("iq3xxs_grid", "IQ3XXS", 4, [4, 12, 20, 28, 36, 44, 52, 62], 3),
    ("iq3s_grid", "IQ3S", 4, [1, 3, 5, 7, 9, 11, 13, 15], 3),
]


def read_table(src, name):
    m = re.search(r"\b" + name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", src, re.S)
    vals = [int(x, 0) for x in re.findall(r"0x[0-9a-fA-F]+|\d+", m.group(2))]
    assert len(vals) == int(m.group(1))
    return vals


def main():
    src = open(REF).read()
    lines = ["// i-quant codebooks as level-index code words; written by tests/golden/make_iq_grids.py (format data of the",
             "// GGUF IQ2 / IQ3 weight types).  Entry e of a table expands to bytes LEVELS[(CODES[e] >> (BITS j)) & mask],",
             "// j = 0 .. bytes-1, little-endian.  Pinned by the SHA-256 of the expanded tables (tests/golden).",
             "// The includer defines IQ_TABLE (e.g. `static const` in C, `static constexpr` in HIP).",
             ""]
    sha = {}
    for ref_name, ours, nb, levels, bits in TABLES:
        vals = read_table(src, ref_name)
        codes, raw = [], bytearray()
        for e in vals:
            c = 0
            for j in range(nb):
                byte = (e >> (8 * j)) & 255
                c |= levels.index(byte) << (bits * j)
                raw.append(byte)
            codes.append(c)
        sha[ours] = {"entries": len(vals), "bytes_per_entry": nb, "sha256": hashlib.sha256(bytes(raw)).hexdigest()}
        lines.append(f"IQ_TABLE uint8_t {ours}_LEVELS[{len(levels)}] = {{{', '.join(map(str, levels))}}};")
        lines.append(f"enum {{ {ours}_BITS = {bits}, {ours}_BYTES = {nb}, {ours}_N = {len(vals)} }};")
        lines.append(f"IQ_TABLE uint16_t {ours}_CODES[{len(vals)}] = {{")
        for i in range(0, len(codes), 16):
            lines.append("    " + ", ".join(f"0x{c:04x}" for c in codes[i:i + 16]) + ",")
        lines.append("};")
        lines.append("")
    open(OUT_INC, "w").write("\n".join(lines))
    json.dump(sha, open(OUT_SHA, "w"), indent=1)
    print("wrote", OUT_INC, OUT_SHA)


if __name__ == "__main__":
    main()
