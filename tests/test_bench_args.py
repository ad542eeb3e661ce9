"""bench.py's argument handling that needs no GPU."""
import bench


def test_bench_measures_one_gpu_only(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err
