"""Writes iq4nl_table.json: the 16 values of the GGUF IQ4_NL / IQ4_XS code table, read as text
from the reference's copy (src/tensor/ggml_tables.h:94-96, `kvalues_iq4nl`).

Run in a container that has the reference at /root/reference: `python tests/golden/make_iq4nl_table.py`.
The JSON it writes is the fixture; the tests read only the JSON.
"""
import json
import re
import sys
from pathlib import Path

SRC = Path("/root/reference/src/tensor/ggml_tables.h")
OUT = Path(__file__).resolve().parent / "iq4nl_table.json"


def main() -> int:
    text = SRC.read_text()
    m = re.search(r"kvalues_iq4nl\s*=\s*\{([^}]*)\}", text)
    if not m:
        print(f"kvalues_iq4nl not found in {SRC}", file=sys.stderr)
        return 1
    vals = [int(v) for v in m.group(1).replace("\n", " ").split(",") if v.strip()]
    if len(vals) != 16:
        print(f"expected 16 values, read {len(vals)}", file=sys.stderr)
        return 1
    line = text[: m.start()].count("\n") + 1
    OUT.write_text(json.dumps({"source": f"src/tensor/ggml_tables.h:{line}", "kvalues_iq4nl": vals}, indent=1) + "\n")
    print(f"wrote {OUT}: {vals}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
