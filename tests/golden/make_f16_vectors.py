"""Writes f16_oracle_vectors.json: the {f32 bits, f16 bits} pairs of the reference's f32->f16 known-answer test.

The pairs are data the reference's own test holds (src/kernels/qsa_oracle_vectors.inc, generated there by numpy's
np.float16(np.float32(x)) and consumed by src/kernels/qsa_parity.cpp:360-405).  This script reads that file as
text in the build container and keeps only the numbers; nothing of the reference is executed.  The GPU box never
reads the reference: it reads the committed JSON.
"""
import json
import re
import sys
from pathlib import Path

SRC = Path("/root/reference/src/kernels/qsa_oracle_vectors.inc")
OUT = Path(__file__).resolve().parent / "f16_oracle_vectors.json"


def main() -> int:
    text = SRC.read_text()
    body = "\n".join(line for line in text.splitlines() if not line.lstrip().startswith("//"))
    values = [int(v, 16) for v in re.findall(r"0x([0-9A-Fa-f]+)u", body)]
    if len(values) % 2:
        raise SystemExit("odd number of values")
    pairs = [[values[i], values[i + 1]] for i in range(0, len(values), 2)]
    OUT.write_text(json.dumps({"source": "src/kernels/qsa_oracle_vectors.inc (numpy float16 of float32)",
                               "pairs_f32_f16": pairs}, separators=(",", ":")) + "\n")
    print(f"wrote {len(pairs)} pairs to {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
