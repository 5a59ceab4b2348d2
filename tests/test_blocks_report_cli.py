"""CPU: the block report's file discovery and text layout (the GPU analysis
itself is tested in test_gpu_blocks_report.py)."""
from __future__ import annotations

from xspmm_amd import blocks_report


def test_mtx_files_expands_directories(tmp_path):
    (tmp_path / "b.mtx").write_text("%%MatrixMarket matrix coordinate real general\n1 1 0\n")
    (tmp_path / "a.mtx").write_text("%%MatrixMarket matrix coordinate real general\n1 1 0\n")
    (tmp_path / "notes.txt").write_text("x")
    files = blocks_report.mtx_files([str(tmp_path), "/some/explicit.mtx"])
    assert [f.split("/")[-1] for f in files] == ["a.mtx", "b.mtx", "explicit.mtx"]


def test_report_text_has_the_reference_summary_lines():
    rec = {"file": "m.mtx", "M": 10, "K": 20, "blocks_before": 8, "blocks_after": 6,
           "blocks_saved": 2, "reduction_pct": 25.0,
           "runs": [{"N": 64, "plan_execute_ms": 0.0123, "plan_tflops": 1.5,
                     "pipeline_ms": {"total_pipeline_ms": 1.0, "clustering_ms": 0.5,
                                     "spmm_ms": 0.01}}]}
    text = blocks_report.report_text(rec)
    lines = text.splitlines()
    assert lines[0] == ">>> Loaded: m.mtx (10x20)"
    assert lines[1].split(":")[1].strip() == "8"
    assert lines[2].split(":")[1].strip() == "6"
    assert "2 blocks (25.00%)" in lines[3]
    assert "N=64" in lines[4] and "prepared execute 0.0123 ms" in lines[4]


def test_cli_without_files_fails_cleanly(tmp_path, capsys):
    assert blocks_report.main([str(tmp_path)]) == 1
    assert "no .mtx files" in capsys.readouterr().err
