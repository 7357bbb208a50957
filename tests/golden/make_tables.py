"""Write tests/golden/ggml_tables.json from the reference's GGML source text.

The tables are data the record formats are defined by; they are read here as
text (nothing of the reference is imported or executed) from
  source/c/ggml/llama.cpp/ggml/src/ggml-common.h
    kmask_iq2xs (:499-501), ksigns_iq2xs (:503-512), iq2xxs_grid (:550-615),
    iq2xs_grid (:617-746), kvalues_mxfp4 (:1116-1118)
and the record sizes from the static_asserts next to each block struct.
Run in the build container:  python tests/golden/make_tables.py
"""
from __future__ import annotations

import json
import re
import sys
from pathlib import Path

REF = Path("/root/reference/source/c/ggml/llama.cpp/ggml/src")
OUT = Path(__file__).resolve().parent / "ggml_tables.json"


def table(text: str, name: str) -> list[int]:
    m = re.search(r"GGML_TABLE_BEGIN\(\s*\w+\s*,\s*" + name + r"\s*,\s*(\d+)\s*\)(.*?)GGML_TABLE_END",
                  text, re.S)
    if not m:
        raise SystemExit(f"table {name} not found")
    body = re.sub(r"//[^\n]*", "", m.group(2))
    vals = [int(tok, 0) for tok in re.findall(r"-?0x[0-9a-fA-F]+|-?\d+", body)]
    if len(vals) != int(m.group(1)):
        raise SystemExit(f"{name}: {len(vals)} values, expected {m.group(1)}")
    return vals


def main() -> int:
    common = (REF / "ggml-common.h").read_text()
    asserts = dict(re.findall(r"static_assert\(sizeof\((block_\w+)\)\s*==\s*([^,]+),", common))
    out = {
        "source": "ggml-common.h of the reference's vendored GGML (read as text)",
        "kmask_iq2xs": table(common, "kmask_iq2xs"),
        "ksigns_iq2xs": table(common, "ksigns_iq2xs"),
        "iq2xxs_grid": [f"{v:016x}" for v in table(common, "iq2xxs_grid")],
        "iq2xs_grid": [f"{v:016x}" for v in table(common, "iq2xs_grid")],
        "kvalues_mxfp4": table(common, "kvalues_mxfp4"),
        "record_size_asserts": {k: asserts[k].strip() for k in
                                ("block_q4_0", "block_mxfp4", "block_q8_0", "block_q4_K",
                                 "block_q8_K", "block_iq2_xxs", "block_q6_K", "block_q5_K", "block_nvfp4",
                                 "block_q4_1", "block_q8_1", "block_iq2_xs")
                                 if k in asserts},
    }
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
