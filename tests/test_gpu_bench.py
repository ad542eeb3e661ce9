"""bench.py's modes run end to end and print one JSON line with the fields the
measurement contract names (short settings; the figures themselves are not
checked here)."""
import json

import pytest

import bench

pytestmark = pytest.mark.gpu

CONTRACT = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config")


def _run(capsys, argv):
    print(f"case bench {' '.join(argv)}", flush=True)
    assert bench.main(argv) == 0
    lines = [ln for ln in capsys.readouterr().out.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, lines
    out = json.loads(lines[0])
    for key in CONTRACT:
        assert key in out, key
    assert out["value"] > 0 and out["n_gpus"] == 1
    return out


def test_attention_bench_with_a_second_window(capsys):
    out = _run(capsys, ["--config", "gt_arxiv", "--steps", "2", "--warmup", "1",
                        "--min-warmup-ms", "0", "--no-cpu", "--also", "gph_slim"])
    assert out["roofline"]["bound"] == "hbm" and 0 < out["roofline"]["frac"] < 1
    slim = out["also"]["gph_slim"]
    assert slim["value"] > 0 and slim["hip_graph_value"] > 0 and slim["dtype"] == "f32"


def test_window_preparation_bench(capsys):
    out = _run(capsys, ["--prep", "--config", "gt_arxiv", "--steps", "1", "--warmup", "0",
                        "--no-cpu"])
    assert out["unit"] == "ms" and out["higher_is_better"] is False


def test_ppr_bench(capsys):
    out = _run(capsys, ["--ppr", "--config", "gt_arxiv", "--no-cpu"])
    assert out["unit"] == "ms" and out["config"]["entries"] > 0
    assert out["config"]["step"] == "direct"
    srt = _run(capsys, ["--ppr", "--config", "gt_arxiv", "--no-cpu", "--ppr-method", "sort"])
    assert srt["config"]["step"] == "sort" and srt["config"]["entries"] == out["config"]["entries"]
    one = _run(capsys, ["--ppr", "--config", "gt_arxiv", "--no-cpu", "--ppr-streams", "1"])
    assert out["config"]["streams"] == 8 and one["config"]["streams"] == 1
    assert one["config"]["entries"] == out["config"]["entries"]
