"""bench.py's command line on the CPU: one GPU only (a request for more exits with a
message and status 2, before any GPU work), and the argument surface the driver uses."""
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]


def run(*args):
    return subprocess.run([sys.executable, str(ROOT / 'bench.py'), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = run('--gpus', '2', '--steps', '5', '--warmup', '1')
    assert r.returncode == 2
    assert 'one GPU' in r.stderr and r.stdout == ''


def test_world_size_above_one_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / 'bench.py')], capture_output=True, text=True, timeout=120,
                       cwd=ROOT, env={'WORLD_SIZE': '2', 'PATH': '/usr/bin:/bin'})
    assert r.returncode == 2 and 'one GPU' in r.stderr


def test_help_lists_the_driver_flags():
    r = run('--help')
    assert r.returncode == 0
    for flag in ('--gpus', '--steps', '--warmup', '--mode', '--no-cpu-baseline'):
        assert flag in r.stdout


def test_event_stride_samples_ten_launches():
    """Per-kernel events in the timed region: the stride never exceeds 8 steps and always
    leaves ten or more sampled launches of each kernel when the run has that many."""
    import importlib.util
    spec = importlib.util.spec_from_file_location('bench_mod', ROOT / 'bench.py')
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for steps in (1, 5, 16, 20, 37, 128, 256):
        for per_step in (1, 2):
            k = bench.event_stride(steps, per_step)
            assert 1 <= k <= bench.EVERY
            sampled = len(range(0, steps, k)) * per_step
            assert sampled >= min(10, steps * per_step), (steps, per_step, k)
    assert bench.event_stride(20, 2) == 4 and bench.event_stride(128, 2) == bench.EVERY
