"""bench.py's contract on the CPU: more than one GPU is refused with a
message (this build measures one GPU), and the prefill CPU-baseline leg
reports what it ran on (a reduced-budget run of the same code)."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_cpu_baseline_prefill_fields(monkeypatch):
    import bench
    from fish_amd import synth
    # a small stand-in for the layer shapes keeps this a unit test; the
    # timing code and the reported fields are the ones bench.py uses
    monkeypatch.setattr(synth, "LAYER_SHAPES", {"qkv": (256, 128), "o": (256, 64)})
    res = bench.cpu_baseline_prefill(0.0)
    for k in ("value", "unit", "cores", "kind", "cpu_model", "build", "sample",
              "m512_g256_layer_TOPS", "m2048_g256_layer_TOPS"):
        assert k in res, k
    assert res["unit"] == "TOP/s" and res["kind"] == "port" and res["cores"] >= 1
    assert res["value"] == res["m2048_g256_layer_TOPS"] > 0
    assert "family" in res["cpu_model"]
