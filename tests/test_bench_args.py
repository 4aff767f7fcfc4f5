"""bench.py's argument handling (CPU only): the counts the driver passes
(`--steps 20 --warmup 5`) and the defaults become whole launches, at least
the steps asked for, and the line reports the steps actually timed."""
import bench


def test_driver_counts_round_up_to_whole_launches():
    a = bench.parse_args(["--gpus", "1", "--steps", "20", "--warmup", "5"])
    n, nw = bench.launches_for(a.steps, a.warmup, a.steps_per_launch)
    assert (n, nw) == (bench.MIN_TIMED_LAUNCHES, bench.MIN_WARMUP_LAUNCHES)
    assert n * a.steps_per_launch >= 20 and nw * a.steps_per_launch >= 5


def test_default_counts():
    a = bench.parse_args([])
    n, nw = bench.launches_for(a.steps, a.warmup, a.steps_per_launch)
    assert a.gpus == 1
    S = a.steps_per_launch
    assert (n * S, nw * S) == (max(16384, bench.MIN_TIMED_LAUNCHES * S),
                               max(1024, bench.MIN_WARMUP_LAUNCHES * S))


def test_counts_are_minimums():
    for steps, warm, s in [(0, 0, 256), (1, 0, 256), (257, 256, 256), (20, 5, 16), (64, 64, 64)]:
        n, nw = bench.launches_for(steps, warm, s)
        assert n >= bench.MIN_TIMED_LAUNCHES and nw >= bench.MIN_WARMUP_LAUNCHES
        assert n * s >= steps and nw * s >= warm
        assert n == bench.MIN_TIMED_LAUNCHES or (n - 1) * s < steps
        assert nw == bench.MIN_WARMUP_LAUNCHES or (nw - 1) * s < warm


def test_cpu_threads_within_the_gpu_share():
    used, visible = bench.host_threads()
    assert 1 <= used <= min(visible, bench.CPU_SHARE)
