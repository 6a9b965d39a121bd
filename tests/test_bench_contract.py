"""bench.py's contract on the CPU: it measures one GPU and refuses --gpus
above 1 (before touching torch or a device), and the headline's byte count --
the numerator of `value` and `roofline.achieved` -- is the sum of the GDN
decode step's algorithmic terms at the reference's shapes (B = 4 sequences,
48 v heads of 128 x 128 fp32 state, a conv of width 4 over the 10240-channel
q|k|v row, fp16 activations)."""
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize("n", [2, 8])
def test_bench_refuses_more_than_one_gpu(n):
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", str(n)],
                       capture_output=True, text=True, timeout=120, cwd=REPO)
    assert r.returncode == 2, r.stdout + r.stderr
    assert f"bench.py measures one GPU: --gpus {n} is not supported" in r.stderr
    assert r.stdout == ""                       # no contract line for a refused run


def test_gdn_decode_bytes_terms():
    sys.path.insert(0, str(REPO))
    import bench
    B, nv, d, row = 4, 48, 128, 10240
    state = 2 * B * nv * d * d * 4              # every state read once and written once
    ring = 2 * B * 3 * row * 2                  # width-4 conv keeps 3 rows, read + write
    x = B * row * 2                             # this step's q|k|v rows
    w = 4 * row * 2                             # conv taps
    gates = 2 * B * nv * 4 + 2 * nv * 4         # a, b per sequence; A_log, dt_bias
    y = B * nv * d * 2
    assert (state, ring, x, w, gates, y) == (25_165_824, 491_520, 81_920, 81_920, 1_920,
                                             49_152)
    assert bench.gdn_decode_bytes() == state + ring + x + w + gates + y == 25_872_256
    # the measured traffic sits just above the algorithmic bytes (no wasted re-reads)
    assert 1.0 <= bench.GDN_DECODE_TRAFFIC_BYTES / bench.gdn_decode_bytes() < 1.1
