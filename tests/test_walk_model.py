"""CPU: the host model of the sip and gulp kernels' reads
(tests/walk_model.cpp) over the library's own plan and cursor code
(drinkme_amd/csrc/plan.h).

The kernels bounds-check no read (the reach pad is the contract, as in
drinkme's src/drinkme/codec/radix_gpu.py:13-27); what keeps their directory
reads inside the array, and every block summed once into the right partial,
is the walk. The model plans every configuration's launches
(the Qwen3-8B and 32B-class groups, lm_head, small and ragged groups, six
hundred seeded random groups) for the sip, gulp, decode and raw-twin kernels
at M = 1..8 and three CU counts, and walks every wave of every workgroup,
past its work as far as a load pipeline runs ahead. It also decodes every
code pattern through the gulp tables as the kernel looks them up (the
tables' entries and lookup are plan.h's, shared with the kernel) against a
direct decode: a layout mistake there only sends blocks down the exact
fallback, correct but slow, so no parity test would see it. The five planted
mistakes are its negative controls: each must be caught."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("walk") / "walk_model")
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror",
                    "-I" + os.path.join(ROOT, "drinkme_amd", "csrc"), "-I" + os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "walk_model.cpp"), "-o", exe], check=True)
    return exe


def test_every_walk_stays_in_range_and_covers_each_block_once(model):
    res = subprocess.run([model], capture_output=True, text=True, timeout=300)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 violations" in res.stdout
    plans = int(res.stdout.split("walk model: ")[1].split(" plans")[0])
    assert plans > 500


@pytest.mark.parametrize("plant", [1, 2, 3, 4, 5])
def test_planted_walk_mistakes_are_caught(model, plant):
    res = subprocess.run([model, "--plant", str(plant)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and "caught" in res.stdout and "NOT" not in res.stdout, res.stdout + res.stderr
