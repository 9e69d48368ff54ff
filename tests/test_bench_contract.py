"""CPU checks of bench.py's contract: one GPU only, the input-set rotation,
the roofline fields and the per-part measured traffic (no GPU needed)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_world_size_above_one_exits(monkeypatch):
    env = dict(os.environ, WORLD_SIZE="4")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True,
                       text=True, timeout=120, env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_sets_must_be_positive():
    r = run_bench("--sets", "0")
    assert r.returncode == 2 and "--sets" in r.stderr


def test_rotating_cycles_through_the_sets_in_order():
    seen = []
    run = bench.rotating([lambda i=i: seen.append(i) or i for i in range(3)])
    assert [run() for _ in range(7)] == [0, 1, 2, 0, 1, 2, 0]
    assert seen == [0, 1, 2, 0, 1, 2, 0]


class _FakeTensor:
    """Counts live output blocks the way the library's allocator would."""
    live = 0
    peak = 0

    def __init__(self, numel):
        self.numel = numel
        _FakeTensor.live += 1
        _FakeTensor.peak = max(_FakeTensor.peak, _FakeTensor.live)

    def __del__(self):
        _FakeTensor.live -= 1


class _FakeCa:
    def synchronize(self):
        pass

    def event_reset(self):
        pass

    def event_record(self):
        return 0

    def event_elapsed(self, a, b):
        return 1.0


@pytest.mark.parametrize("out_mib,numel,blocks", [(512, 16 << 20, 8), (512, 32 << 20, 4),
                                                  (0, 16 << 20, 1), (512, 1000, 1),
                                                  (512, 1 << 18, 64)])
def test_timed_rotates_output_blocks(monkeypatch, out_mib, numel, blocks):
    """Outputs of 1 MiB or more stay alive so that `blocks` of them rotate
    (512 MiB of 64 MiB outputs: 8), every block exists before the timed
    steps, and all are released at the end; --out-mib 0 reuses one block."""
    monkeypatch.setattr(bench, "OUT_HOLD_BYTES", out_mib << 20)
    _FakeTensor.live = _FakeTensor.peak = 0
    calls = []

    def launch():
        calls.append(_FakeTensor.live)  # blocks alive when this step allocates
        return [_FakeTensor(numel)]

    bench.timed(_FakeCa(), launch, steps=30, warmup=2)
    assert _FakeTensor.peak == blocks
    assert _FakeTensor.live == 0
    timed_calls = calls[-30:]
    assert all(c == blocks - 1 for c in timed_calls)
    assert len(calls) - 30 >= blocks  # the warmup allocated every block


def test_roofline_fields():
    r = bench.roofline("hbm", 6000.0, 8000.0, "GB/s", 123)
    assert r == {"bound": "hbm", "achieved": 6000.0, "peak": 8000.0, "unit": "GB/s",
                 "frac": 0.75, "traffic": 123}
    assert bench.roofline("mfma", 100.0, bench.FP32_MFMA_PEAK_TFS, "TFLOP/s")["frac"] == \
        round(100.0 / 157.3, 4)


def test_part_traffic_sums_the_parts_kernels(tmp_path):
    kernels = {k: {"bytes_per_launch": 100 * (i + 1)}
               for i, k in enumerate(bench.PART_KERNELS["mse"])}
    path = tmp_path / "traffic.json"
    path.write_text(json.dumps({"kernels": kernels}))
    out = {"mse": {"roofline": bench.roofline("hbm", 1.0, 8000.0, "GB/s")},
           "matmul_4096": {"roofline": bench.roofline("mfma", 1.0, 157.3, "TFLOP/s")},
           "softmax": {"roofline": bench.roofline("hbm", 1.0, 8000.0, "GB/s")}}
    bench.add_part_traffic(out, str(path))
    assert out["mse"]["roofline"]["traffic"] == sum(v["bytes_per_launch"]
                                                    for v in kernels.values())
    assert out["matmul_4096"]["roofline"]["traffic"] is None  # MFMA-bound: no traffic
    assert out["softmax"]["roofline"]["traffic"] is None      # its kernel is not in the file


@pytest.mark.parametrize("name", sorted(bench.PART_KERNELS))
def test_committed_traffic_summary_covers_every_part(name):
    """profiles/hbm_traffic.json names every kernel the HBM-bound parts
    launch, so each part's roofline.traffic is filled from measurement."""
    with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
        kernels = json.load(f)["kernels"]
    missing = [k for k in bench.PART_KERNELS[name] if k not in kernels]
    assert not missing, f"{name}: {missing} not in profiles/hbm_traffic.json"


def test_check_parity_records_pass_and_failure(monkeypatch):
    """A part within |g - c| <= atol + rtol |c| is "ok"; one element past the
    bound, a shape mismatch or a NaN is reported as a failure."""
    monkeypatch.setattr(bench, "PARITY", {})
    want = [1.0, -2.0, 100.0]
    bench.check_parity("inside", [1.0 + 1.2e-6, -2.0, 100.0 - 1e-4], want, 1e-6, 5e-7)
    bench.check_parity("outside", [1.0, -2.0 - 1e-3, 100.0], want, 1e-6, 5e-7)
    bench.check_parity("shape", [1.0, -2.0], want, 1e-6, 5e-7)
    bench.check_parity("nan", [1.0, float("nan"), 100.0], want, 1e-6, 5e-7)
    bench.check_parity("exact", [1.0, -2.0, 100.0], want, 0.0, 0.0)
    assert bench.PARITY["inside"] == "ok"
    assert bench.PARITY["exact"] == "ok"
    assert bench.PARITY["outside"].startswith("1 of 3 elements")
    assert bench.PARITY["shape"].startswith("shape")
    assert bench.PARITY["nan"].startswith("1 of 3 elements")
