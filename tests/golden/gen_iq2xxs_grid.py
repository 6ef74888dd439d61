"""Writes tests/golden/iq2xxs_grid.json: the IQ2_XXS grid of the reference,
read as text (not executed) from /root/reference/js/quant-tables.js:40-105,
the `IQ2XXS_GRID = new Uint32Array([...])` literal: 512 u32 words, word 2e
holding bytes 0..3 of entry e and word 2e + 1 bytes 4..7 (little-endian).

The fixture is data (a format table); the oracle loads it as its grid, and
tests/test_oracle.py checks the product's csrc/iq2xxs_grid.inc against it.
Run in the build container, where the reference is present:
    python tests/golden/gen_iq2xxs_grid.py
"""
import json
import os
import re
import sys

SRC = "/root/reference/js/quant-tables.js"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "iq2xxs_grid.json")


def main():
    text = open(SRC, encoding="utf-8").read()
    m = re.search(r"export const IQ2XXS_GRID = new Uint32Array\(\[(.*?)\]\);", text, re.S)
    if not m:
        sys.exit("IQ2XXS_GRID literal not found")
    start = text[:m.start()].count("\n") + 1
    end = text[:m.end()].count("\n") + 1
    words = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{8})\b", m.group(1))]
    if len(words) != 512:
        sys.exit(f"expected 512 words, found {len(words)}")
    doc = {"source": f"js/quant-tables.js:{start}-{end} (IQ2XXS_GRID)",
           "layout": "512 u32; entry e, weight j (0..7) = byte j % 4 of word 2e + j / 4 (little-endian)",
           "words": words}
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=0)
        f.write("\n")
    print(f"wrote {OUT}: 512 words from lines {start}-{end}")


if __name__ == "__main__":
    main()
