"""bench.py's roofline.traffic (no GPU): the committed PMC figure is reported
only while the kernel's sources are the ones it was measured on."""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def write(tmp_path, rec):
    p = tmp_path / "traffic.json"
    p.write_text(json.dumps(rec))
    return str(p)


def test_matching_sources_report_the_figure(tmp_path):
    op = "gelu_tanh_bias"
    p = write(tmp_path, {op: 123, "_sources_sha256": {op: bench.traffic_sources_sha(op)}})
    assert bench.measured_traffic(op, p) == (123, False)


def test_changed_sources_report_null(tmp_path):
    op = "qk_rmsnorm_rope"
    p = write(tmp_path, {op: 456, "_sources_sha256": {op: "0" * 64}})
    assert bench.measured_traffic(op, p) == (None, True)
    p = write(tmp_path, {op: 456})   # no fingerprint recorded: cannot vouch for it
    assert bench.measured_traffic(op, p) == (None, True)


def test_missing_file_or_op(tmp_path):
    assert bench.measured_traffic("ln_modulate", str(tmp_path / "absent.json")) == (None, False)
    p = write(tmp_path, {"_sources_sha256": {}})
    assert bench.measured_traffic("ln_modulate", p) == (None, False)


def test_fingerprint_covers_each_source():
    # every op's fingerprint names existing files, and ops on different
    # kernels get different fingerprints
    shas = {op: bench.traffic_sources_sha(op) for op in bench.TRAFFIC_SOURCES}
    assert shas["gelu_tanh_bias"] == shas["gate_residual"]   # one source file
    assert len({shas["ln_modulate"], shas["qk_rmsnorm_rope"], shas["gelu_tanh_bias"]}) == 3
