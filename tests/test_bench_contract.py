"""CPU checks of bench.py's contract pieces that need no GPU: the one-GPU
refusal, the committed traffic summary the roofline reads, and the
roofline arithmetic."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    """--gpus N > 1 exits with status 2 and says why, before touching a GPU."""
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2, r
    assert "one GPU" in r.stderr and r.stdout == "", r


def test_traffic_summary_covers_the_bench_lines():
    """Every key the bench line's roofline reads from profiles/traffic.txt is
    there: the headline config, and the decode GEMV defaults at C3."""
    head = bench.traffic_of("gemm_i8_4096_dequant_f16:256x256_w2x4")
    assert head is not None and 64e6 < head < 300e6, head
    for m in (1, 4, 16):
        t = bench.traffic_of(f"gemv_w8a16_m{m}:gemv_packed_ct3_kw16_e")
        assert t is not None and 45e6 < t < 60e6, (m, t)
    assert bench.traffic_of("no_such_kernel") is None


def test_roofline_fraction():
    r = bench.roofline("hbm", 4000.0, bench.PEAK_HBM_GBS, "GB/s", 123)
    assert r == {"bound": "hbm", "achieved": 4000.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.5, "traffic": 123}
