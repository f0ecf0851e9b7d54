"""Regenerate the golden fixtures: ``python tests/golden/make_fixtures.py``.

Writes ``<case>.npz`` for every case of ``cases.CASES`` and
``manifest.json`` beside this file.  Runs the float64 oracle on the CPU
(a few seconds).
"""

from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

from golden import cases, store  # noqa: E402


def main():
    man = {}
    for name, (make_in, make_out, seed) in cases.CASES.items():
        x = make_in(seed)
        man[name] = store.save(name, seed, x, make_out(x))
        kib = os.path.getsize(store.path(name)) / 1024
        print(f"{name}: {kib:.0f} KiB", flush=True)
    with open(store.MANIFEST, "w") as f:
        json.dump(man, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
