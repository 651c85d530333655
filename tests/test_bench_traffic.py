"""bench.py reports a kernel's measured HBM traffic (profiles/traffic.json)
only while the kernel's sources hash to the digest recorded with the
measurement, so `roofline.traffic` always describes the kernel that ran."""
import json
import os

import bench


def write_entry(tmp_path, sources, digest, traffic=12345):
    p = tmp_path / "traffic.json"
    p.write_text(json.dumps({"k": {"kernel": "x", "commit": "0", "sources": sources, "source_sha256": digest,
                                   "traffic_bytes": traffic}}))
    return str(p)


def test_traffic_reported_while_the_sources_match(tmp_path, monkeypatch):
    srcs = ["qx_amd/csrc/common.h"]
    monkeypatch.setattr(bench, "TRAFFIC_FILE", write_entry(tmp_path, srcs, bench.source_digest(srcs)))
    assert bench.load_traffic("k") == 12345


def test_traffic_withheld_after_a_source_change(tmp_path, monkeypatch):
    srcs = ["qx_amd/csrc/common.h"]
    monkeypatch.setattr(bench, "TRAFFIC_FILE", write_entry(tmp_path, srcs, "0" * 64))
    assert bench.load_traffic("k") is None


def test_traffic_withheld_for_unknown_or_legacy_entries(tmp_path, monkeypatch):
    p = tmp_path / "traffic.json"
    p.write_text(json.dumps({"legacy": 2158894973}))
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(p))
    assert bench.load_traffic("legacy") is None
    assert bench.load_traffic("missing") is None


def test_digest_covers_file_names_and_contents(tmp_path, monkeypatch):
    a, b = tmp_path / "a.h", tmp_path / "b.h"
    a.write_text("x")
    b.write_text("x")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    da, db = bench.source_digest(["a.h"]), bench.source_digest(["b.h"])
    assert da != db  # same contents, different file
    b.write_text("y")
    assert bench.source_digest(["a.h", "b.h"]) == bench.source_digest(["b.h", "a.h"])  # order-free


def test_committed_entries_name_their_kernel_commit_and_sources():
    with open(os.path.join(bench.ROOT, "profiles", "traffic.json")) as f:
        entries = json.load(f)
    for key in ("cfg4_decode", "cfg5a_decode", "kvhash"):
        e = entries[key]
        assert e["kernel"].startswith("qxh::") and e["commit"] and e["sources"]
        assert len(e["source_sha256"]) == 64 and e["traffic_bytes"] > e["algorithmic_bytes"] * 0.99
