"""CPU checks of bench.py's contract: the one-GPU refusal for --gpus N > 1
(before anything touches a device), the algorithmic byte counts the JSON
line is computed from, and the parser of the driver's clock tables."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_algorithmic_bytes():
    import bench
    # config 5 GQA layer at L = 32768: K and V once, q and out once
    assert bench.gqa_bytes(8, 16, 4, 256, 32768) == 2 * 8 * 4 * 32768 * 256 * 2 + 2 * 8 * 16 * 256 * 2
    assert bench.gqa_bytes(8, 16, 4, 256, 32768) == 1_073_872_896
    # config 1: 2,105,344 bytes per call
    assert bench.gqa_bytes(1, 16, 8, 128, 512) == 2_105_344
    # config 3 state traffic: 2 * 33,554,432 bytes of fp32 state per step plus activations
    b3 = bench.deltanet_bytes(32, 16, 16, 128, 128)
    assert 2 * 33_554_432 < b3 < 2 * 33_554_432 + 1_000_000


@pytest.mark.parametrize("text,levels,cur", [
    ("S: 99Mhz *\n0: 500Mhz\n1: 2400Mhz\n", [500, 2400], 99),     # idle: sleep level current
    ("0: 500Mhz\n1: 174Mhz *\n2: 2400Mhz\n", [500, 2400], 174),   # between levels: extra starred line
    ("0: 500Mhz\n1: 1994Mhz *\n", [500], 1994),                   # under load: the top level reads the clock
    ("0: 2000Mhz *\n", [2000], 2000),                             # memory clock, one level
    ("", [], None),
])
def test_dpm_table_parser(tmp_path, text, levels, cur):
    import bench
    p = tmp_path / "pp_dpm"
    p.write_text(text)
    assert bench._dpm_levels(str(p)) == (levels, cur)
