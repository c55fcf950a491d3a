"""Host-side pieces of bench.py: the rule that ties the committed HBM-traffic record to the decode
kernels it was counted on, and the one-GPU contract."""

from __future__ import annotations

import json
import subprocess
import sys

import bench


def test_traffic_record_applies_to_the_current_decode_code_only(monkeypatch, tmp_path) -> None:
    record = json.loads((bench.REPO / bench.TRAFFIC_RECORD).read_text())
    alg = record["algorithmic_bytes_per_call"]
    assert record["decode_source_sha256"] == bench.decode_source_sha256()
    assert bench.measured_traffic(alg) == record["traffic_bytes_per_call"]
    assert bench.measured_traffic(alg + 1) is None  # another shape

    code = (bench.REPO / bench.DECODE_SOURCE).read_text()
    src = tmp_path / "decode.hip"
    monkeypatch.setattr(bench, "REPO", tmp_path)
    monkeypatch.setattr(bench, "DECODE_SOURCE", "decode.hip")
    (tmp_path / "profiles").mkdir()
    (tmp_path / bench.TRAFFIC_RECORD).write_text(json.dumps(record))
    # Comments, blank lines and trailing spaces do not change the kernels.
    src.write_text("// a note\n" + code.replace("\n", "  \n\n") + "\n/* another\n note */\n")
    assert bench.measured_traffic(alg) == record["traffic_bytes_per_call"]
    # Any change of code does.
    src.write_text(code.replace("kDeepRowsOf = D == 128 ? 256 : 120;", "kDeepRowsOf = D == 128 ? 255 : 120;"))
    assert "? 255 : 120;" in src.read_text()
    assert bench.measured_traffic(alg) is None


def test_more_than_one_gpu_is_refused_with_a_message() -> None:
    r = subprocess.run([sys.executable, str(bench.REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert "exactly one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
