"""bench.py's command line on the CPU (no GPU needed): more than one GPU is
refused with a message and exit status 2 before anything touches a device,
and the arguments the driver and the profiles pass parse."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_arguments_parse():
    sys.path.insert(0, ROOT)
    import bench
    argv = sys.argv
    try:
        sys.argv = ["bench.py", "--config", "3", "--m", "3", "--no-cpu", "--no-traffic", "--no-fixed", "--steps", "5",
                    "--warmup", "1"]
        a = bench.parse()
    finally:
        sys.argv = argv
    assert (a.config, a.m, a.no_cpu, a.no_traffic, a.no_fixed, a.steps, a.warmup) == (3, 3, True, True, True, 5, 1)
    assert a.gpus == 1
