"""bench.py's launch plans, built on the CPU for the command lines the bench is run with."""
import subprocess
import sys

import pytest

import bench


@pytest.mark.parametrize("argv", [
    ["--gpus", "1", "--steps", "20", "--warmup", "5"],
    [],
    ["--steps", "7", "--warmup", "0", "--layers", "3", "--int4-steps", "50", "--layer-steps", "11"],
    ["--steps", "1", "--warmup", "1", "--layers", "48"],
])
def test_every_leg_plan_stays_inside_the_token_rows(argv):
    args = bench.parse_args(argv)
    steps = bench.leg_steps(args)
    assert set(steps) == {"decode", "layer", "int4"}
    rows = bench.token_rows(args.layers, args.warmup, steps)
    for leg, n in steps.items():
        plan = bench.step_plan(args.layers, args.warmup, n)
        assert len(plan) == args.warmup + n
        assert all(0 <= l < args.layers and 0 <= r < rows for l, r in plan), leg
        # consecutive steps move to another layer (the rotation the bench relies on)
        if args.layers > 1:
            assert all(a[0] != b[0] for a, b in zip(plan, plan[1:]))


def test_driver_command_times_the_requested_steps():
    args = bench.parse_args(["--gpus", "1", "--steps", "20", "--warmup", "5"])
    assert bench.leg_steps(args) == {"decode": 20, "layer": 20, "int4": 20}


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                       cwd=bench.os.path.dirname(bench.os.path.abspath(bench.__file__)))
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_host_cpu_fields():
    model, phys, logical, usable = bench.host_cpu()
    assert isinstance(model, str) and model
    assert logical >= 1 and 1 <= usable <= logical
    assert phys is None or 1 <= phys <= logical
    assert 1 <= bench.cpu_threads(usable) <= 16


def test_algorithmic_bytes_of_the_workloads():
    from tarfa_amd.moe import MoEShape
    full = MoEShape(2560, 256, 1024, 8, 1024)
    assert bench.decode_bytes(full) == 142_873_600
    assert bench.decode_bytes(MoEShape(1024, 32, 512, 8, 0)) == 25_231_360
    assert bench.decode_bytes_int4(full) == 8 * 4_055_040 + 15_728_640 + 1_310_720 + 5_120
    assert bench.prefill_weight_bytes(full) == 4_026_531_840 + 15_728_640
