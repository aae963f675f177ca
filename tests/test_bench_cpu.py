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


def test_bench_traffic_and_bytes_follow_the_instance():
    """The headline is the drop-in O-only call: its roofline reads the O-only traffic line of the
    committed counter summary and counts no LSE bytes; the O + LSE leg reads its own line."""
    bench = _bench()
    o_only = bench.committed_traffic()
    with_lse = bench.committed_traffic("traffic_bytes_per_launch")
    assert o_only is not None and with_lse is not None
    # measured fabric traffic is at least the algorithmic bytes of each instance
    assert o_only >= bench.bytes_per_fwd(lse=False)
    assert with_lse >= bench.bytes_per_fwd(lse=True)
    B, H, N, D = bench.B, bench.H, bench.N, bench.D
    assert bench.bytes_per_fwd(lse=False) == 2 * 4 * B * H * N * D
    assert bench.bytes_per_fwd(lse=True) == 2 * 4 * B * H * N * D + 4 * B * H * N
    assert bench.committed_traffic("no_such_key") is None
