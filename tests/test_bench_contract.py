"""bench.py's output contract: one JSON line with the metric, the timing
and the two objects measured beside it (roofline, cpu_baseline), the
algorithmic byte count it prices every GEMV at, the workloads it sweeps,
and its refusals (more than one GPU; no GPU)."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _run(*args, timeout=600):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    res = _run("--gpus", "2", timeout=300)
    assert res.returncode != 0
    assert "one GPU" in res.stderr


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU may be present")
def test_no_gpu_exits_cleanly():
    res = _run("--workload", "linear-4096", "--steps", "1", "--warmup", "0", timeout=300)
    assert res.returncode == 1 and "needs a GPU" in res.stderr
    assert res.stdout.strip() == ""


def test_algorithmic_bytes_is_the_stated_formula():
    # B = 4 NW + 4 (R NB + 1) + P + 2 M C + 2 M R, P = 7 (sip) / 21 (gulp)
    rt = {"R": 3, "C": 2100, "block_size": 1024, "NW": 1234, "profile": "sip"}
    nb = 3
    assert bench.algorithmic_bytes(rt, 1) == 4 * 1234 + 4 * (3 * nb + 1) + 7 + 2 * 2100 + 2 * 3
    rt["profile"] = "gulp"
    assert bench.algorithmic_bytes(rt, 4) == 4 * 1234 + 4 * (3 * nb + 1) + 21 + 2 * 4 * 2100 + 2 * 4 * 3


def test_workloads_hold_the_configured_gemvs():
    step = bench.workload_items("qwen3-8b-step")
    assert len(step) == 36 * 7 + 1 and step[-1][3:5] == (151936, 4096)
    assert sum(r * c for _, _, _, r, c, _ in step) == 7568097280
    assert len(bench.workload_items("qwen3-8b-layer")) == 4 * 7
    assert len(bench.workload_items("32b-layer")) == 2 * 7
    lin = bench.workload_items("linear-4096")
    assert len(lin) == 32 and {(r, c) for _, _, _, r, c, _ in lin} == {(4096, 4096)}


@pytest.mark.gpu
def test_the_json_line_carries_the_contract():
    res = _run("--workload", "linear-4096", "--steps", "5", "--warmup", "2")
    assert res.returncode == 0, res.stderr[-2000:]
    lines = [ln for ln in res.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, "bench prints exactly one line to stdout"
    out = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 5 and out["warmup"] == 2
    assert out["unit"] == "GB/s" and out["higher_is_better"] is True and out["value"] > 0
    assert out["config"]["workload"] == "linear-4096"
    # value is the sweep's algorithmic bytes over its time
    c = out["config"]
    assert abs(out["value"] - c["compressed_bytes"] / (out["ms_per_step"] * 1e-3) / 1e9) <= 0.01 * out["value"]
    for k in ("ungrouped", "eager_ungrouped", "eager_modules"):
        assert c[k]["us_per_sweep"] > 0 and c[k]["launches"] >= 1, k
    # the plain read of the same launches: a ceiling for the same bytes, so
    # no faster than the HBM peak, and the sweep's share of it below 1.1
    rw = c["read_wall"]
    assert 0 < rw["value"] < 8000.0 and 0 < rw["largest_launch"]["value"] < 8000.0
    assert 0 < rw["sweep_fraction_of_read_wall"] < 1.1
    assert rw["per_launch_kind"], "every launch kind timed against its plain read"
    for name, pk in rw["per_launch_kind"].items():
        assert pk["launches"] >= 1 and pk["kernel_us"] > 0 and pk["read_us"] > 0, name
        assert abs(pk["kernel_over_read"] - pk["kernel_us"] / pk["read_us"]) < 0.01, name
    r = out["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    assert abs(r["achieved"] - r["bytes_per_launch"] / (r["us_per_launch"] * 1e-6) / 1e9) <= 0.01 * r["achieved"]
    assert r["settle_replays"] > 0
    cb = out["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample", "legs"):
        assert key in cb, key
    assert set(cb["legs"]) == {"cpu_share", "one_thread", "cached_w"}
    assert cb["nproc"] >= 1 and 1 <= cb["cores"] <= min(cb["affinity_cpus"], 16)
    assert cb["legs"]["one_thread"]["cores"] == 1 and cb["kind"] in ("reference", "port")
