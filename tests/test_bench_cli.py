"""bench.py's command-line contract on the CPU: one GPU only, and every workload line labelled.

The measurements themselves need a GPU (bench.py exits with status 1 without one); what is checked here is
what a driver relies on before any GPU work: the refusal of several GPUs, the default workload's metric
being BASELINE.json's, and each workload naming its own metric.
"""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          cwd=ROOT, env=env, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="4")
    r = run_bench(env=env)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_default_workload_reports_the_baseline_metric():
    sys.path.insert(0, ROOT)
    import bench
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        base = json.load(f)
    assert bench.METRIC == base["metric"]
    assert bench.WORKLOADS[bench.extra_workloads()] is bench.Stack
    assert getattr(bench.Stack, "metric", bench.METRIC) == base["metric"]


def test_every_workload_has_a_name_and_its_own_metric():
    sys.path.insert(0, ROOT)
    import bench
    seen = set()
    for key, W in bench.WORKLOADS.items():
        assert W.name == key
        m = getattr(W, "metric", bench.METRIC)
        if W is not bench.Stack:
            assert m != bench.METRIC, key  # a single-kernel line must not carry the headline label
        assert m not in seen, key
        seen.add(m)
