"""Write the validation record that gates loading libsmx.so.

Runs the repository's GPU test suite (``pytest tests -m gpu``) against the
library as built, and on completion writes a JSON record

  {"complete": true, "library": "libsmx.so", "library_sha256": "...",
   "code_objects_sha256": {"libsmx.<source>.co": "...", ...},
   "abi_version": N, "pytest": {"exit": 0, "passed": P, "failed": 0,
   "errors": 0, "skipped": S}, "created": "..."}

which ``native.load()`` checks before loading the library
(check_validation_record: complete, this ABI version, no failure, the
library's sha256) -- the record the environment variable
SMX_VALIDATION_RECORD names, else libsmx.validation.json beside the library
(the default --record) -- and the step runner before it loads the device
code objects (check_code_objects).  The
reference deploys its kernel library the same way: a validation run writes
head-validation.json with the library's digest, and the loader refuses the
library unless the record is complete and the digest matches
(src/spark_vllm_ascend/integration/head.py:22-27).

Usage (on a machine with the GPU, from anywhere):
  python spark-vllm-ascend_amd/native/validate.py [--record /path/validation.json]
"""
from __future__ import annotations

import argparse
import datetime
import json
import os
import subprocess
import sys
import tempfile
import xml.etree.ElementTree as ET
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
LIB = HERE / "libsmx.so"


def _abi_version() -> int:
    src = (HERE / "__init__.py").read_text()
    for line in src.splitlines():
        if line.startswith("ABI_VERSION"):
            return int(line.split("=")[1])
    raise RuntimeError("ABI_VERSION not found")


def _junit_counts(path: Path) -> dict:
    root = ET.parse(path).getroot()
    suites = [root] if root.tag == "testsuite" else list(root.iter("testsuite"))
    c = {"tests": 0, "failed": 0, "errors": 0, "skipped": 0}
    for s in suites:
        c["tests"] += int(s.get("tests", 0))
        c["failed"] += int(s.get("failures", 0))
        c["errors"] += int(s.get("errors", 0))
        c["skipped"] += int(s.get("skipped", 0))
    c["passed"] = c["tests"] - c["failed"] - c["errors"] - c["skipped"]
    return c


def make_record(pytest_exit: int, counts: dict, lib: Path = LIB, code_objects=None) -> dict:
    import hashlib
    if code_objects is None:
        sys.path.insert(0, str(HERE))
        try:
            from build import code_object_paths
        finally:
            sys.path.pop(0)
        code_objects = [p for p in code_object_paths() if p.exists()]
    return {"complete": True, "library": lib.name,
            "library_sha256": hashlib.sha256(lib.read_bytes()).hexdigest(),
            "code_objects_sha256": {Path(p).name: hashlib.sha256(Path(p).read_bytes()).hexdigest()
                                    for p in code_objects},
            "abi_version": _abi_version(),
            "pytest": {"exit": int(pytest_exit), "passed": counts["passed"],
                       "failed": counts["failed"], "errors": counts["errors"],
                       "skipped": counts["skipped"]},
            "created": datetime.datetime.now(datetime.timezone.utc).isoformat()}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--record", default=str(LIB.with_name("libsmx.validation.json")),
                    help="where to write the JSON record (default: beside the library, "
                         "where native.load() looks for it)")
    ap.add_argument("--pytest-args", default="", help="extra pytest arguments")
    args = ap.parse_args(argv)
    if not LIB.exists():
        print(f"{LIB} is not built", file=sys.stderr)
        return 2
    with tempfile.TemporaryDirectory() as tmp:
        junit = Path(tmp) / "junit.xml"
        cmd = [sys.executable, "-m", "pytest", str(REPO / "tests"), "-m", "gpu", "-q",
               f"--junitxml={junit}", *args.pytest_args.split()]
        # the run validates the library as built: no record vouches for it yet
        env = {k: v for k, v in os.environ.items() if k != "SMX_VALIDATION_RECORD"}
        env["SMX_ALLOW_UNVALIDATED"] = "1"
        rc = subprocess.run(cmd, cwd=REPO, env=env).returncode
        if not junit.exists():
            print("pytest wrote no results; no record written", file=sys.stderr)
            return rc or 1
        counts = _junit_counts(junit)
    rec = make_record(rc, counts)
    Path(args.record).write_text(json.dumps(rec, indent=1) + "\n")
    print(f"wrote {args.record}: {rec['pytest']}")
    return 0 if rc == 0 else rc


if __name__ == "__main__":
    sys.exit(main())
