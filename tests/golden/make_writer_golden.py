#!/usr/bin/env python3
"""Writes writer_golden.json: the length and sha256 of the file that writer_case.write
produces on the reference's own writer, tools/convert.py's Writer (lines 128-262).

Runs in the build container only, where the reference tree is readable; tools/convert.py
needs numpy and the standard library alone. The result is committed, so the test that
compares this repository's writer with it (tests/test_rlm.py) needs no reference code.

    python tests/golden/make_writer_golden.py [/root/reference]
"""

from __future__ import annotations

import hashlib
import importlib.util
import json
import os
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import writer_case  # noqa: E402


def main() -> None:
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    spec = importlib.util.spec_from_file_location("reference_convert", os.path.join(ref, "tools", "convert.py"))
    convert = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(convert)
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "model")
        os.makedirs(src)
        for name, data in writer_case.FILES.items():
            with open(os.path.join(src, name), "wb") as fh:
                fh.write(data)
        path = os.path.join(tmp, "golden.rlm")
        writer_case.write(convert.Writer(path), lambda w: w.add_files(src))
        data = open(path, "rb").read()
    out = {"source": "tools/convert.py Writer (the reference), run by tests/golden/make_writer_golden.py",
           "case": "tests/golden/writer_case.py", "seed": writer_case.SEED,
           "bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}
    with open(os.path.join(HERE, "writer_golden.json"), "w") as fh:
        json.dump(out, fh, indent=1)
        fh.write("\n")
    print(json.dumps(out))


if __name__ == "__main__":
    main()
