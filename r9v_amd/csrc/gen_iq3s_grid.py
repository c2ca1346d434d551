"""Writes r9vx_iq3s_grid.h: the IQ3_S codebook (512 entries of 4 odd values
1..15), a table of the GGUF format itself that every IQ3_S decoder must hold
unchanged.

Source: the reference's gguf-py 0.19.0-derived table
crates/r9v-format/src/iq_lut.rs:629-630 (IQ3_S_GRID, 2048 u8, entry e = values
4e..4e+3).  Run once where /root/reference exists; the header is committed.
Checks before writing: the reference's own facts (crates/r9v-format/tests/iq.rs:505,
514-516: 2048 values, all odd and <= 15) and that the 512 little-endian words
ascend strictly (the llama.cpp table is sorted, so a dropped, doubled or
swapped entry fails).  Each word packs entry e's values, value b in byte b.
"""
import pathlib
import re
import sys

SRC = pathlib.Path("/root/reference/crates/r9v-format/src/iq_lut.rs")
DST = pathlib.Path(__file__).resolve().parent / "r9vx_iq3s_grid.h"


def main() -> int:
    text = SRC.read_text()
    m = re.search(r"pub const IQ3_S_GRID: \[u8; 2048\] = \[(.*?)\];", text, re.S)
    vals = [int(t) for t in re.findall(r"\d+", m.group(1))]
    assert len(vals) == 2048 and all(v % 2 == 1 and v <= 15 for v in vals)
    words = [vals[4 * e] | vals[4 * e + 1] << 8 | vals[4 * e + 2] << 16 | vals[4 * e + 3] << 24 for e in range(512)]
    assert all(words[i] < words[i + 1] for i in range(511))
    out = ["/* r9vx_iq3s_grid.h -- the GGUF IQ3_S codebook: 512 entries of four odd",
           " * values in 1..15, entry e in word e with value b in byte b (the table of",
           " * crates/r9v-format/src/iq_lut.rs:629-630, gguf-py 0.19.0 IQ3_S.grid).",
           " * Written by gen_iq3s_grid.py; the words ascend strictly. */",
           "#ifndef R9VX_IQ3S_GRID_H", "#define R9VX_IQ3S_GRID_H", "",
           "#include <stdint.h>", "",
           "#define R9VX_IQ3S_GRID_WORDS \\"]
    for i in range(0, 512, 8):
        sep = ", \\" if i + 8 < 512 else ""
        out.append("    " + ", ".join(f"0x{w:08x}u" for w in words[i:i + 8]) + sep)
    out += ["", "#endif", ""]
    DST.write_text("\n".join(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
