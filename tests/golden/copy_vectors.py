"""Copies the reference's own decode vectors (data files, not code) into this directory.

    python tests/golden/copy_vectors.py

Source: cozy-runtime's `src/cozy_runtime/internal/encoding/vectors/cases/{name}.json`, read as
JSON text from `/root/reference` (present only where this build was made; nothing at test time
reads it). Each output keeps the source's cases whose component is a scheme this build decodes,
plus every refusal case of those files, unchanged, under a `source` note.
"""

from __future__ import annotations

import json
from pathlib import Path

SOURCE = Path("/root/reference/src/cozy_runtime/internal/encoding/vectors/cases")
HERE = Path(__file__).resolve().parent
#: file -> the components kept (refusal cases are kept for every file)
KEEP = {
    "int8": {"int8.convrot", "int8.rowwise", "int8.tensorwise", "int8.columnwise"},
    "fp8": {"fp8.rowwise", "fp8.tensorwise", "fp8.columnwise"},
    "mxfp8": {"mxfp8"},
    "nvfp4": {"nvfp4"},
    "svdq": {"svdq"},
}


def main() -> None:
    for name, components in KEEP.items():
        data = json.loads((SOURCE / f"{name}.json").read_text())
        cases = [c for c in data["cases"] if c["component"] in components | {"refuse"}]
        out = {"source": f"cozy_runtime/internal/encoding/vectors/cases/{name}.json",
               "cases": cases}
        (HERE / f"ref_{name}_vectors.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
        print(f"{name}: {len(cases)} of {len(data['cases'])} cases")


if __name__ == "__main__":
    main()
