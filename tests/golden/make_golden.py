"""Writes the golden fixtures (tests/golden/*.json) from the oracle.

    python tests/golden/make_golden.py [case ...]

Every case is defined in ``cases.py``; this script only runs it on the
oracle backend it names and stores the record.  Rerun it only when a case
definition changes, and commit the JSON with the change.
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # repo root: oracle, nanoinfer_amd
sys.path.insert(0, os.path.dirname(HERE))                   # tests/: the golden package

from golden import cases  # noqa: E402


def main(names):
    for name in names or list(cases.CASES):
        rec = cases.CASES[name](cases.oracle_backend(name))
        path = os.path.join(HERE, f"{name}.json")
        with open(path, "w") as f:
            json.dump(rec, f)
            f.write("\n")
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1:])
