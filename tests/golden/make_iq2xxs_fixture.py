"""Writes iq2xxs_tables.json: the IQ2_XXS codebook (256 entries of 8 bytes)
and sign table (128 entries) as the reference holds them, read as text from
rsllm-gguf/src/dequant/iq2_xxs/tables.rs (KSIGNS_IQ2XS at :26, IQ2XXS_GRID at
:43; both GGUF format constants). Run in a checkout with the reference tree:

    python tests/golden/make_iq2xxs_fixture.py [/root/reference]

The fixture is data (the two tables); tests/test_golden_iq2xxs.py checks the
oracle's and the HIP library's decoders against it."""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REL = "crates/rsllm-gguf/src/dequant/iq2_xxs/tables.rs"


def parse(text: str):
    def array(name):
        m = re.search(r"const\s+" + name + r"\s*:\s*\[[^\]]+\]\s*=\s*\[(.*?)\];", text, re.S)
        if not m:
            raise ValueError(f"{name} not found")
        body = re.sub(r"//[^\n]*", "", m.group(1))
        return [int(t, 0) for t in re.findall(r"0x[0-9a-fA-F]+|\d+", body)]
    grid = array("IQ2XXS_GRID")
    signs = array("KSIGNS_IQ2XS")
    if len(grid) != 256 or len(signs) != 128:
        raise ValueError(f"unexpected table sizes {len(grid)}, {len(signs)}")
    return grid, signs


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    grid, signs = parse(open(os.path.join(ref, REL)).read())
    out = {"source": REL + " (KSIGNS_IQ2XS :26, IQ2XXS_GRID :43)",
           "grid": [f"0x{v:016x}" for v in grid], "ksigns": signs}
    path = os.path.join(HERE, "iq2xxs_tables.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
