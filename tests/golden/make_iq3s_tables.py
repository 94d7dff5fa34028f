"""Writes iq3s_tables.json: the two tables of the GGUF IQ3_S format, read as text from the
reference's copy (src/tensor/ggml_tables.h): `iq3s_grid` (512 packed 4-byte codebook entries)
and `kmask_iq2xs` (the 8 sign-bit masks).

Run in a container that has the reference at /root/reference:
`python tests/golden/make_iq3s_tables.py`. The JSON it writes is the fixture; the tests read
only the JSON.
"""
import json
import re
import sys
from pathlib import Path

SRC = Path("/root/reference/src/tensor/ggml_tables.h")
OUT = Path(__file__).resolve().parent / "iq3s_tables.json"


def table(text: str, name: str, n: int):
    m = re.search(name + r"\s*=\s*\{([^}]*)\}", text)
    if not m:
        raise SystemExit(f"{name} not found in {SRC}")
    vals = [int(v, 0) for v in m.group(1).replace("\n", " ").split(",") if v.strip()]
    if len(vals) != n:
        raise SystemExit(f"{name}: expected {n} values, read {len(vals)}")
    return vals, text[: m.start()].count("\n") + 1


def main() -> int:
    text = SRC.read_text()
    grid, gl = table(text, "iq3s_grid", 512)
    mask, ml = table(text, "kmask_iq2xs", 8)
    OUT.write_text(json.dumps({"source": {"iq3s_grid": f"src/tensor/ggml_tables.h:{gl}",
                                          "kmask_iq2xs": f"src/tensor/ggml_tables.h:{ml}"},
                               "kmask_iq2xs": mask, "iq3s_grid": grid}) + "\n")
    print(f"wrote {OUT}: {len(grid)} grid entries, masks {mask}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
