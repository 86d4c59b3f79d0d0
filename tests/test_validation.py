"""The validation-gated load of libsmx.so (CPU): native.load() refuses the
library unless a record vouches for it -- the one SMX_VALIDATION_RECORD
names, else the default record beside the library; complete, this ABI
version, a GPU test run without failures, the library's sha256 -- as the
reference refuses its kernel library without a complete validation record
whose digest matches (src/spark_vllm_ascend/integration/head.py:22-27).
Only SMX_ALLOW_UNVALIDATED=1 (what this suite, the benchmark and the build
check set) loads an unvalidated library."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

from _util import pkg

ROOT = Path(__file__).resolve().parent.parent


def _record(tmp_path, **over):
    native = pkg("native")
    validate = pkg("native.validate")
    rec = validate.make_record(0, {"passed": 350, "failed": 0, "errors": 0, "skipped": 6},
                               native.LIB_PATH)
    for k, v in over.items():
        if k.startswith("pytest_"):
            rec["pytest"][k[7:]] = v
        else:
            rec[k] = v
    path = tmp_path / "validation.json"
    path.write_text(json.dumps(rec))
    return path


def test_record_for_this_library_is_accepted(tmp_path):
    native = pkg("native")
    path = _record(tmp_path)
    assert native.check_validation_record(path) == native.library_sha256()
    assert json.loads(path.read_text())["abi_version"] == native.ABI_VERSION


@pytest.mark.parametrize("over,why", [
    ({"complete": False}, "not complete"),
    ({"abi_version": 1}, "ABI"),
    ({"library_sha256": "0" * 64}, "sha256"),
    ({"pytest_exit": 1}, "did not all pass"),
    ({"pytest_failed": 2}, "did not all pass"),
    ({"pytest_errors": 1}, "did not all pass"),
    ({"pytest_passed": 0}, "no GPU test passed"),
])
def test_bad_records_are_rejected(tmp_path, over, why):
    native = pkg("native")
    with pytest.raises(RuntimeError, match=why):
        native.check_validation_record(_record(tmp_path, **over))


def test_missing_or_garbled_record(tmp_path):
    native = pkg("native")
    with pytest.raises(RuntimeError, match="unreadable"):
        native.check_validation_record(tmp_path / "absent.json")
    bad = tmp_path / "bad.json"
    bad.write_text("{not json")
    with pytest.raises(RuntimeError, match="unreadable"):
        native.check_validation_record(bad)


def test_record_of_another_library_is_rejected(tmp_path):
    native = pkg("native")
    other = tmp_path / "libsmx.so"
    other.write_bytes(native.LIB_PATH.read_bytes() + b"\0")
    with pytest.raises(RuntimeError, match="sha256"):
        native.check_validation_record(_record(tmp_path), other)


@pytest.mark.parametrize("good", [True, False])
def test_load_is_gated_by_the_environment(tmp_path, good):
    """In a fresh process (load() caches the library): with the variable set,
    load() succeeds only when the record vouches for the library."""
    path = _record(tmp_path, **({} if good else {"library_sha256": "f" * 64}))
    code = ("import __graft_entry__ as g; g.load_package(); "
            "import spark_vllm_ascend_amd.native as n; n.load(); print('loaded')")
    env = dict(os.environ, SMX_VALIDATION_RECORD=str(path))
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=300)
    if good:
        assert res.returncode == 0 and "loaded" in res.stdout, res.stderr
    else:
        assert res.returncode != 0 and "rejected" in res.stderr


def test_record_vouches_for_the_runner_code_objects(tmp_path):
    """The step runner loads the device code objects beside the library: the
    record carries their digests, and a changed or missing one is refused."""
    native = pkg("native")
    paths = [tmp_path / "libsmx.a.co", tmp_path / "libsmx.b.co"]
    for i, p in enumerate(paths):
        p.write_bytes(bytes([i]) * 64)
    validate = pkg("native.validate")
    rec = validate.make_record(0, {"passed": 1, "failed": 0, "errors": 0, "skipped": 0},
                               native.LIB_PATH, code_objects=paths)
    path = tmp_path / "validation.json"
    path.write_text(json.dumps(rec))
    native.check_code_objects(path, paths)
    paths[1].write_bytes(b"\1" * 65)
    with pytest.raises(RuntimeError, match="libsmx.b.co"):
        native.check_code_objects(path, paths)
    with pytest.raises(RuntimeError, match="libsmx.c.co"):
        native.check_code_objects(path, [paths[0], tmp_path / "libsmx.c.co"])


def test_default_record_lists_the_built_code_objects(tmp_path):
    native = pkg("native")
    build = pkg("native.build")
    rec = pkg("native.validate").make_record(
        0, {"passed": 1, "failed": 0, "errors": 0, "skipped": 0}, native.LIB_PATH)
    assert set(rec["code_objects_sha256"]) == {p.name for p in build.code_object_paths()}


def _load_in_fresh_process(env):
    code = ("import __graft_entry__ as g; g.load_package(); "
            "import spark_vllm_ascend_amd.native as n; n.load(); print('loaded', n.checked_record())")
    return subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                          text=True, timeout=300)


def test_load_requires_a_record_by_default():
    """No variable set and no record beside the library: load() refuses and
    says how to validate; SMX_ALLOW_UNVALIDATED=1 loads it unchecked."""
    native = pkg("native")
    if native.DEFAULT_RECORD.exists():
        pytest.skip("a validation record sits beside the library on this machine")
    env = {k: v for k, v in os.environ.items()
           if k not in ("SMX_VALIDATION_RECORD", "SMX_ALLOW_UNVALIDATED")}
    res = _load_in_fresh_process(env)
    assert res.returncode != 0 and "no validation record" in res.stderr, res.stderr[-2000:]
    assert "validate.py" in res.stderr
    res = _load_in_fresh_process(dict(env, SMX_ALLOW_UNVALIDATED="1"))
    assert res.returncode == 0 and "loaded None" in res.stdout, res.stderr[-2000:]


def test_a_named_record_is_checked_even_when_unvalidated_loads_are_allowed(tmp_path):
    path = _record(tmp_path, library_sha256="e" * 64)
    env = dict(os.environ, SMX_VALIDATION_RECORD=str(path), SMX_ALLOW_UNVALIDATED="1")
    res = _load_in_fresh_process(env)
    assert res.returncode != 0 and "rejected" in res.stderr
