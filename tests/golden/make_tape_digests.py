"""Writes tests/golden/tape_digests.json: for each benchmark tape, the SHA-256
of its canonical wire bytes (nablatensor_amd.rocm.TapeArrays.wire_bytes) and
of the HIP source nt_lower emits for it with default options in fp64 and fp32.

The tape digests pin the recorder and the wire format; the source digests pin
the lowering. A foreign-function adapter (the Java binding) checks the same
two values for the arrays it marshals: equal tape digest, then equal source
digest from nt_lower. Rerun this script after an intended change of the
recorder or the lowering:

    python tests/golden/make_tape_digests.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))


def digests() -> dict:
    from nablatensor_amd import rocm, workloads

    out = {}
    for name, tape in workloads.workload_tapes().items():
        flat = tape.flat()
        row = {"nodes": int(len(flat["op"])), "tape_sha256": rocm.wire_digest(flat)}
        for precision in ("fp64", "fp32"):
            src = rocm.lower(flat, rocm.options(precision))
            row[f"source_sha256_{precision}"] = hashlib.sha256(src.encode()).hexdigest()
        out[name] = row
    return out


def main() -> None:
    doc = {"_about": "SHA-256 of each benchmark tape's wire bytes and of its lowered HIP source "
                     "(default options); written by tests/golden/make_tape_digests.py. Data only.",
           **digests()}
    path = Path(__file__).resolve().parent / "tape_digests.json"
    path.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
