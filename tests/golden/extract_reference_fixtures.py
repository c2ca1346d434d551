"""Copies the reference's own golden decode vectors for this path into tests/golden.

Data only (inputs and expected outputs); run once in the build container where
/root/reference exists.  Sources:
  crates/r9v-format/tests/fixtures/r9v-format/q4k_reference.txt  (all 6 Q4_K cases,
      consumed by crates/r9v-format/tests/schemes.rs:482-516)
  crates/r9v-format/tests/fixtures/r9v-format/iq_a24_reference.txt (the IQ4_XS,
      IQ4_NL and IQ3_S cases, consumed by crates/r9v-format/tests/iq.rs:159-197)
  crates/r9v-format/tests/fixtures/r9v-format/gguf_a23_reference.txt (the Q8_0, Q6_K
      and Q4_K cases, consumed by crates/r9v-format/tests/gguf.rs:44-90,172-180)
      -> gguf_a23_reference.txt
  crates/r9v-format/tests/fixtures/r9v-format/{a25_standard,a25_split-0000{1,2}-of-00002,
      llama_tiny_q80}.hex (whole GGUF files as hex text, consumed by
      crates/r9v-format/tests/container.rs:72-330, 897-930) -> tests/golden/gguf/
The reference is Apache-2.0; the fixture data derives from llama.cpp / gguf-py (MIT).
"""
import pathlib
import sys

SRC = pathlib.Path("/root/reference/crates/r9v-format/tests/fixtures/r9v-format")
DST = pathlib.Path(__file__).resolve().parent

HEADER = ("# Copied verbatim (data lines) from R9V {src} -- reference golden vectors.\n"
          "# License: Apache-2.0 (R9V); data derived from llama.cpp / gguf-py (MIT).\n")


def main() -> int:
    q4k = (SRC / "q4k_reference.txt").read_text()
    (DST / "q4k_reference.txt").write_text(
        HEADER.format(src="crates/r9v-format/tests/fixtures/r9v-format/q4k_reference.txt") + q4k)
    keep, out = False, []
    for line in (SRC / "iq_a24_reference.txt").read_text().splitlines():
        if line.startswith("#"):
            out.append(line)
            continue
        if line.startswith("case "):
            keep = line.split()[1] in ("IQ4_XS", "IQ4_NL", "IQ3_S")
        if keep:
            out.append(line)
    (DST / "iq4_reference.txt").write_text(
        HEADER.format(src="crates/r9v-format/tests/fixtures/r9v-format/iq_a24_reference.txt")
        + "\n".join(out) + "\n")
    keep, out = False, []
    for line in (SRC / "gguf_a23_reference.txt").read_text().splitlines():
        if line.startswith("#"):
            out.append(line)
            continue
        if line.startswith("case "):
            keep = line.split()[1] in ("Q8_0", "Q6_K", "Q4_K")
        if keep:
            out.append(line)
    (DST / "gguf_a23_reference.txt").write_text(
        HEADER.format(src="crates/r9v-format/tests/fixtures/r9v-format/gguf_a23_reference.txt")
        + "\n".join(out) + "\n")
    gdir = DST / "gguf"
    gdir.mkdir(exist_ok=True)
    for name in ("a25_standard", "a25_split-00001-of-00002", "a25_split-00002-of-00002",
                 "llama_tiny_q80"):
        src = f"crates/r9v-format/tests/fixtures/r9v-format/{name}.hex"
        (gdir / f"{name}.hex").write_text(
            HEADER.format(src=src) + (SRC / f"{name}.hex").read_text().strip() + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
