"""bench.py's host side, no GPU: the config table its timed legs use equals the oracle's, and
it refuses more than one GPU before touching torch."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_config_table_matches_oracle():
    from oracle import CONFIGS

    bench = _bench()
    assert set(bench.BENCH_CONFIGS) == set(CONFIGS)
    for name, c in CONFIGS.items():
        b = bench.BENCH_CONFIGS[name]
        assert (b.B, b.H, b.N, b.D, b.sigma_qk, b.sigma_v, b.seed) == (
            c.B, c.H, c.N, c.D, c.sigma_qk, c.sigma_v, c.seed), name
        assert (b.flops, b.bytes, b.scale) == (c.flops, c.bytes, c.scale), name
    # the headline workload is config 3
    c3 = bench.BENCH_CONFIGS["config3"]
    assert (bench.B, bench.H, bench.N, bench.D, bench.SIGMA_QK, bench.SIGMA_V) == (
        c3.B, c3.H, c3.N, c3.D, c3.sigma_qk, c3.sigma_v)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_bench_rejects_unknown_profile_workload_before_touching_the_gpu():
    r = subprocess.run([sys.executable, BENCH, "--profile", "config3,config9"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "config9" in r.stderr
