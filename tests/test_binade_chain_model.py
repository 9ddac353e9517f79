"""CPU model of the whole-vocabulary sampler's exact parallel running sums
(`binade_chain_model.c`: the block algorithm of sample.hip's
sample_full_kernel restated in C) against one-after-another f32 sums, the
order prepareProbabilities and sampleCandidate add in
(src/generator.zig:428-463). Bit-identical on every input; each of three
planted mistakes in the algorithm must be caught. The device kernel itself is
compared with sequential sums in tests/test_gpu_sampling.py."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).with_name("binade_chain_model.c")


def _build(tmp_path, *flags):
    exe = tmp_path / ("model" + "".join(f.replace("-D", "_") for f in flags))
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", *flags, "-o", str(exe), str(SRC), "-lm"], check=True)
    return exe


@pytest.fixture(scope="module")
def gcc():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    return True


def test_model_matches_sequential_sums(gcc, tmp_path):
    r = subprocess.run([str(_build(tmp_path)), "240"], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    ties = int(r.stdout.split(" mismatched, ")[1].split(" ties")[0])
    assert ties > 10000  # the inputs include runs of exact ties


@pytest.mark.parametrize("flag", ["-DDROP_FLIP", "-DDROP_INPUT_FLIP", "-DDROP_TIES"])
def test_planted_mistakes_are_caught(gcc, tmp_path, flag):
    r = subprocess.run([str(_build(tmp_path, flag)), "80"], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0, f"{flag} went unnoticed: {r.stdout}"
