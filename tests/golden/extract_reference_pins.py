"""Write tests/golden/reference_pins.json from the reference's own test data.

The reference pins four real GGUF blocks (two Q4_K, two Q6_K) taken from the
Ornith 9B Q4_K_M file, with values computed by gguf-py's independent
dequantizer (crates/unltd-tensor/src/quants.rs:1094-1152 bytes,
:1169-1198 expected values, x formulas :1157-1166). This script reads that
file as text and stores the byte arrays and expected values as a JSON
fixture; it runs none of the reference's code.

Usage: python tests/golden/extract_reference_pins.py [/path/to/reference]
"""
import json
import os
import re
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
SRC = os.path.join(REF, "crates/unltd-tensor/src/quants.rs")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_pins.json")


def main():
    text = open(SRC, encoding="utf-8").read()
    blocks = {}
    for name, n, body in re.findall(r"const (\w+): \[u8; (\d+)\] = \[(.*?)\];", text, re.S):
        vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{2})", body)]
        assert len(vals) == int(n), (name, len(vals), n)
        blocks[name] = vals
    m = re.search(r"let cases: \[\(&\[u8\], f64, f64, f64, f64\); 4\] = \[(.*?)\];", text, re.S)
    cases = []
    for name, nums in re.findall(r"\(\s*&(\w+),(.*?)\)", m.group(1), re.S):
        vals = [float(v) for v in re.findall(r"-?\d+\.\d+(?:e-?\d+)?", nums)]
        assert len(vals) == 4, (name, vals)
        cases.append({"block": name, "dot_x_pattern": vals[0], "dot_x_alt": vals[1],
                      "w7": vals[2], "w200": vals[3]})
    fixture = {
        "source": "crates/unltd-tensor/src/quants.rs:1094-1222 (ornith_decode_pin)",
        "tolerance": 1e-4,
        "x_pattern": "((i * 7919) % 1009) as f32 / 1009.0 - 0.5, i in 0..256 (f32 arithmetic)",
        "x_alt": "((i * 31 + 17) % 257) as f32 / 257.0 - 0.5, i in 0..256 (f32 arithmetic)",
        "blocks": {k: {"dtype": "Q6_K" if len(v) == 210 else "Q4_K", "bytes": v}
                   for k, v in blocks.items()},
        "cases": cases,
    }
    with open(OUT, "w") as f:
        json.dump(fixture, f, indent=1)
    print(f"wrote {OUT}: {len(blocks)} blocks, {len(cases)} cases")


if __name__ == "__main__":
    main()
