"""Result envelopes for benchmark measurements (version 1).

The envelope is the reference's portable result format
(src/sfu_repro/artifact.py, schemas/result-v1.json): a JSON object with
`schema_version` (= 1), `experiment` (`id` matching ``[a-z0-9][a-z0-9._-]*``,
optional description, provenance class, UTC creation time and command),
`source`, `environment` and `measurement` metadata objects, and `results`,
either a list of observations (`case`, `variant`, `workload`, `metrics`,
`samples`) or an object.  The checks below restate that schema's
constraints without a JSON-schema library (none is installed on the MI355X
image); like the reference's validator, the messages name the location and
the rule, never the offending value.
"""

from __future__ import annotations

import argparse
import datetime as _dt
import json
import re
from pathlib import Path
from typing import Any

SCHEMA_VERSION = 1
PROVENANCE_CLASSES = (
    "new-measurement",
    "diagnostic-unbound-source",
    "historical-materialized",
    "historical-source-derived",
    "blocked",
)
_ID = re.compile(r"^[a-z0-9][a-z0-9._-]*$")
_SHA1 = re.compile(r"^[0-9a-f]{40}$")
_SHA256 = re.compile(r"^[0-9a-f]{64}$")
_REQUIRED = ("schema_version", "experiment", "source", "environment", "measurement", "results")


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _is_num(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _is_datetime(v) -> bool:
    if not isinstance(v, str) or "T" not in v:
        return False
    try:
        _dt.datetime.fromisoformat(v.replace("Z", "+00:00"))
    except ValueError:
        return False
    return True


class _Checker:
    def __init__(self) -> None:
        self.errors: list[str] = []

    def fail(self, loc: str, rule: str) -> None:
        self.errors.append(f"{loc}: {rule}")

    def typed(self, loc: str, value, kinds: tuple, name: str) -> bool:
        ok = any(k(value) for k in kinds)
        if not ok:
            self.fail(loc, f"must have type {name}")
        return ok

    def optional_fields(self, loc: str, obj: dict, spec: dict) -> None:
        for key, (kinds, name) in spec.items():
            if key in obj:
                self.typed(f"{loc}.{key}", obj[key], kinds, name)


_STR = (lambda v: isinstance(v, str),)
_STR_NULL = (lambda v: isinstance(v, str), lambda v: v is None)
_BOOL_NULL = (lambda v: isinstance(v, bool), lambda v: v is None)
_INT_NULL = (_is_int, lambda v: v is None)
_OBJ = (lambda v: isinstance(v, dict),)


def validate_result(document: Any) -> list[str]:
    """Value-blind failures of `document` against the version-1 envelope."""
    c = _Checker()
    if not isinstance(document, dict):
        c.fail("$", "must have type object")
        return c.errors
    missing = sorted(k for k in _REQUIRED if k not in document)
    if missing:
        c.fail("$", "missing required field(s): " + ", ".join(missing))
    if "schema_version" in document and (not _is_int(document["schema_version"])
                                         or document["schema_version"] != SCHEMA_VERSION):
        c.fail("$.schema_version", "violates the const constraint")

    exp = document.get("experiment")
    if exp is not None and c.typed("$.experiment", exp, _OBJ, "object"):
        if "id" not in exp:
            c.fail("$.experiment", "missing required field(s): id")
        elif c.typed("$.experiment.id", exp["id"], _STR, "string"):
            if not exp["id"]:
                c.fail("$.experiment.id", "violates the minLength constraint")
            elif not _ID.match(exp["id"]):
                c.fail("$.experiment.id", "must match the required pattern")
        c.optional_fields("$.experiment", exp, {"description": (_STR, "string")})
        if "provenance_class" in exp and exp["provenance_class"] not in PROVENANCE_CLASSES:
            c.fail("$.experiment.provenance_class", "violates the enum constraint")
        if "created_utc" in exp and c.typed("$.experiment.created_utc", exp["created_utc"], _STR, "string"):
            if not _is_datetime(exp["created_utc"]):
                c.fail("$.experiment.created_utc", "must be a date-time")
        if "command" in exp and c.typed("$.experiment.command", exp["command"],
                                        (lambda v: isinstance(v, list),), "array"):
            for i, item in enumerate(exp["command"]):
                c.typed(f"$.experiment.command[{i}]", item, _STR, "string")

    src = document.get("source")
    if src is not None and c.typed("$.source", src, _OBJ, "object"):
        c.optional_fields("$.source", src, {
            "repository": (_STR, "string"), "dirty": (_BOOL_NULL, "boolean or null"),
            "git_worktree_dirty": (_BOOL_NULL, "boolean or null"),
            "untracked_files": (_INT_NULL, "integer or null")})
        if "revision" in src and c.typed("$.source.revision", src["revision"], _STR_NULL, "string or null"):
            if isinstance(src["revision"], str) and not _SHA1.match(src["revision"]):
                c.fail("$.source.revision", "must match the required pattern")
        if _is_int(src.get("untracked_files")) and src["untracked_files"] < 0:
            c.fail("$.source.untracked_files", "violates the minimum constraint")
        if "git_revision" in src and c.typed("$.source.git_revision", src["git_revision"], _STR, "string"):
            if not src["git_revision"]:
                c.fail("$.source.git_revision", "violates the minLength constraint")
        for key in ("external_components", "input_sha256"):
            if key in src and c.typed(f"$.source.{key}", src[key], _OBJ, "object"):
                for name, value in src[key].items():
                    loc = f"$.source.{key}.{name}"
                    if key == "input_sha256":
                        if c.typed(loc, value, _STR, "string") and not _SHA256.match(value):
                            c.fail(loc, "must match the required pattern")
                    else:
                        c.typed(loc, value, _STR_NULL, "string or null")

    env = document.get("environment")
    if env is not None and c.typed("$.environment", env, _OBJ, "object"):
        c.optional_fields("$.environment", env, {
            k: (_STR_NULL, "string or null") for k in
            ("gpu", "device_name", "python", "torch", "cuda", "torch_version", "cuda_version", "driver")})
        if "total_memory_bytes" in env and c.typed("$.environment.total_memory_bytes", env["total_memory_bytes"],
                                                   _INT_NULL, "integer or null"):
            if _is_int(env["total_memory_bytes"]) and env["total_memory_bytes"] < 0:
                c.fail("$.environment.total_memory_bytes", "violates the minimum constraint")
        if "sm_clock_mhz" in env and c.typed("$.environment.sm_clock_mhz", env["sm_clock_mhz"],
                                             (_is_num, lambda v: v is None), "number or null"):
            if _is_num(env["sm_clock_mhz"]) and env["sm_clock_mhz"] <= 0:
                c.fail("$.environment.sm_clock_mhz", "violates the exclusiveMinimum constraint")
        if "compute_capability" in env:
            cc = env["compute_capability"]
            pair = isinstance(cc, list) and len(cc) == 2 and all(_is_int(x) and x >= 0 for x in cc)
            if not (cc is None or isinstance(cc, str) or pair):
                c.fail("$.environment.compute_capability", "violates the oneOf constraint")
        if "packages" in env and c.typed("$.environment.packages", env["packages"], _OBJ, "object"):
            for name, value in env["packages"].items():
                c.typed(f"$.environment.packages.{name}", value, _STR_NULL, "string or null")

    meas = document.get("measurement")
    if meas is not None and c.typed("$.measurement", meas, _OBJ, "object"):
        c.optional_fields("$.measurement", meas, {
            "dtype": (_STR, "string"), "seed": (_INT_NULL, "integer or null"),
            "summary_statistic": (_STR, "string"), "order_policy": (_STR, "string")})
        for key, low in (("warmup", 0), ("iterations", 1), ("rounds", 1)):
            if key in meas and c.typed(f"$.measurement.{key}", meas[key], (_is_int,), "integer"):
                if meas[key] < low:
                    c.fail(f"$.measurement.{key}", "violates the minimum constraint")

    res = document.get("results")
    if res is not None:
        if isinstance(res, list):
            for i, obs in enumerate(res):
                loc = f"$.results[{i}]"
                if not c.typed(loc, obs, _OBJ, "object"):
                    continue
                c.optional_fields(loc, obs, {"case": (_STR, "string"), "variant": (_STR, "string"),
                                             "workload": (_OBJ, "object"), "metrics": (_OBJ, "object")})
                if "samples" in obs and c.typed(f"{loc}.samples", obs["samples"],
                                                (lambda v: isinstance(v, list),), "array"):
                    for j, s in enumerate(obs["samples"]):
                        c.typed(f"{loc}.samples[{j}]", s, (_is_num,), "number")
        elif not isinstance(res, dict):
            c.fail("$.results", "violates the oneOf constraint")
    return sorted(c.errors)


def load_and_validate(path: Path) -> list[str]:
    try:
        document = json.loads(Path(path).read_text(encoding="utf-8"))
    except (OSError, json.JSONDecodeError) as error:
        return [str(error)]
    return validate_result(document)


def make_result(experiment_id: str, *, description: str, command: list[str], environment: dict,
                measurement: dict, results: list[dict], source: dict | None = None,
                provenance_class: str = "new-measurement") -> dict:
    """A version-1 envelope around `results` (a list of observations)."""
    return {
        "schema_version": SCHEMA_VERSION,
        "experiment": {
            "id": experiment_id,
            "description": description,
            "provenance_class": provenance_class,
            "created_utc": _dt.datetime.now(_dt.timezone.utc).isoformat(timespec="seconds").replace("+00:00", "Z"),
            "command": list(command),
        },
        "source": dict(source or {}),
        "environment": dict(environment),
        "measurement": dict(measurement),
        "results": list(results),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("paths", type=Path, nargs="+")
    args = parser.parse_args()
    failed = False
    for path in args.paths:
        failures = load_and_validate(path)
        if failures:
            failed = True
            for failure in failures:
                print(f"FAIL {path}: {failure}")
        else:
            print(f"PASS {path}")
    return int(failed)


if __name__ == "__main__":
    raise SystemExit(main())
