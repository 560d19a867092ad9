"""bench.py's output contract: one JSON line with the fields the driver reads, roofline and
cpu_baseline objects, and a refusal of more than one GPU."""

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run(*args, timeout=300):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=timeout)


def _json_line(stdout):
    lines = [ln for ln in stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, stdout
    return json.loads(lines[0])


def test_more_than_one_gpu_is_refused():
    """One GPU only: --gpus 2 exits with status 2 and says so, before touching a device."""
    r = _run("--gpus", "2", timeout=120)
    assert r.returncode == 2, (r.returncode, r.stderr[-2000:])
    line = _json_line(r.stdout)
    assert "one GPU" in line["error"]


@pytest.mark.gpu
def test_json_line_fields():
    """A short headline-config run prints one line with the contract's fields."""
    r = _run("--steps", "3", "--warmup", "1", "--cpu-seconds", "0.5", "--configs", "c1,c3,v2",
             "--sub-steps", "3", "--sub-cpu-seconds", "0.2")
    assert r.returncode == 0, r.stderr[-3000:]
    line = _json_line(r.stdout)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 3 and line["warmup"] == 1
    assert line["value"] > 0 and line["unit"] == "GB/s" and line["higher_is_better"] is True
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["peak"] == 8000.0 and roof["unit"] == "GB/s"
    assert 0 < roof["frac"] <= 1 and abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    cpu = line["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["cores"] >= 1 and cpu["kind"] in ("port", "reference")
    assert isinstance(cpu["sample"], str) and cpu["sample"]
    assert "workload" in line["config"]
    assert line["parity"]["unexplained"] == 0
    # the roofline is taken on the timed region's clock
    assert roof["kernel_ms"] <= line["ms_per_step"]
    subs = line["configs"]
    assert set(subs) == {"c1", "c3", "v2"}
    for name, entry in subs.items():
        assert entry["ms_per_step"] > 0 and entry["cpu_baseline"]["value"] > 0, name
        assert [f["cores"] for f in entry["cpu_baseline"]["by_cores"]][-1] == 1, name
        assert entry["parity"]["mismatched"] == 0 or name == "v2", name
    assert subs["c1"]["frac_on_kernel_bytes"] > 0
    assert subs["c1"]["reference_algorithm_bytes"] > 0 and subs["c1"]["kernel_bytes"] > 0
    assert subs["v2"]["parity"]["unexplained"] == 0
