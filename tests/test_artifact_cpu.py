"""The version-1 result envelope (sfu_repro.artifact, restating the
reference's schemas/result-v1.json constraints) and the envelope bench.py
writes with --rows-out.  CPU only: the bench's environment block is passed
in instead of read from the device."""

import argparse
import copy
import json
import os
import sys

import pytest

from sfu_repro import artifact

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _minimal():
    return {"schema_version": 1, "experiment": {"id": "b1-silu"}, "source": {}, "environment": {},
            "measurement": {}, "results": []}


def test_minimal_envelope_is_valid():
    assert artifact.validate_result(_minimal()) == []


@pytest.mark.parametrize("mutate,message", [
    (lambda d: d.pop("results"), "$: missing required field(s): results"),
    (lambda d: d.update(schema_version=2), "$.schema_version: violates the const constraint"),
    (lambda d: d["experiment"].update(id="B1 SiLU"), "$.experiment.id: must match the required pattern"),
    (lambda d: d["experiment"].update(id=""), "$.experiment.id: violates the minLength constraint"),
    (lambda d: d["experiment"].pop("id"), "$.experiment: missing required field(s): id"),
    (lambda d: d["experiment"].update(provenance_class="guess"),
     "$.experiment.provenance_class: violates the enum constraint"),
    (lambda d: d["experiment"].update(created_utc="yesterday"), "$.experiment.created_utc: must be a date-time"),
    (lambda d: d["experiment"].update(command=["bench.py", 3]), "$.experiment.command[1]: must have type string"),
    (lambda d: d["source"].update(revision="abc"), "$.source.revision: must match the required pattern"),
    (lambda d: d["source"].update(untracked_files=-1), "$.source.untracked_files: violates the minimum constraint"),
    (lambda d: d["source"].update(input_sha256={"x": "00"}), "$.source.input_sha256.x: must match the required pattern"),
    (lambda d: d["environment"].update(total_memory_bytes="big"),
     "$.environment.total_memory_bytes: must have type integer or null"),
    (lambda d: d["environment"].update(compute_capability=[9]),
     "$.environment.compute_capability: violates the oneOf constraint"),
    (lambda d: d["measurement"].update(iterations=0), "$.measurement.iterations: violates the minimum constraint"),
    (lambda d: d["measurement"].update(warmup=True), "$.measurement.warmup: must have type integer"),
    (lambda d: d.update(results=[{"samples": [1.0, "x"]}]), "$.results[0].samples[1]: must have type number"),
    (lambda d: d.update(results="none"), "$.results: violates the oneOf constraint"),
])
def test_violations_are_reported_without_values(mutate, message):
    doc = _minimal()
    mutate(doc)
    errors = artifact.validate_result(doc)
    assert message in errors, errors


def test_load_and_validate_reads_files(tmp_path):
    good = tmp_path / "good.json"
    good.write_text(json.dumps(_minimal()))
    bad = tmp_path / "bad.json"
    bad.write_text("{not json")
    assert artifact.load_and_validate(good) == []
    assert len(artifact.load_and_validate(bad)) == 1


def test_bench_rows_envelope_is_valid():
    sys.path.insert(0, ROOT)
    import bench

    rows = [{"function": "softcap_tanh_d4", "config": "C3", "dtype": "bf16", "elements": 8,
             "bytes_per_launch": 32, "poly_us": 1.0, "native_us": 1.1, "speedup": 1.1,
             "poly_numerics": {"max_abs": 0.4, "max_ulp": 21, "max_rel": 0.09}},
            {"function": "stream_ceiling", "elements": 8, "unit": "fraction of 8 TB/s", "copy": 0.8}]
    headline = {"metric": "m", "value": 1.0, "config": {"workload": "C3", "elements": 8}, "configs": {}}
    args = argparse.Namespace(warmup=5, sweep_reps=100)
    env = {"gpu": "AMD Instinct MI355X", "device_name": "AMD Instinct MI355X", "python": "3.10",
           "torch_version": "2.10", "cuda_version": None, "total_memory_bytes": 1 << 38,
           "packages": {"numpy": "2.2"}}
    doc = bench.result_envelope(rows, headline, args, env)
    assert artifact.validate_result(doc) == []
    assert [o["case"] for o in doc["results"]] == ["headline", "softcap_tanh_d4", "stream_ceiling"]
    assert doc["results"][1]["workload"]["config"] == "C3"
    assert doc["results"][1]["metrics"]["poly_us"] == 1.0
    broken = copy.deepcopy(doc)
    broken["experiment"]["id"] = "MI355X bench"
    assert artifact.validate_result(broken) == ["$.experiment.id: must match the required pattern"]
