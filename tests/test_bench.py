"""bench.py's host-side pieces (no GPU): the algorithmic bytes per world-step (the survey's compulsory-traffic
formula), the traffic figure read from the committed profile summaries, the TOI-tail statistics of a State, and the
refusal of more than one GPU."""
import importlib.util
import subprocess
import sys
from pathlib import Path

import numpy as np

from util import b2, wd

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
bench = importlib.util.module_from_spec(spec)
spec.loader.exec_module(bench)


def test_bytes_per_world_step():
    # R = 113B + 24F_d + 54J + 93C + 21, W = 81B + 16F_d + 28J + 120C + 17
    assert bench.bytes_per_world_step(5, 4, 3, 32) == 3820 + 4410  # the rig at 32 slots: 8,230 B
    assert bench.bytes_per_world_step(5, 4, 3, 40) == 9934          # the headline workload's 40 slots
    assert bench.bytes_per_world_step(17, 16, 3, 64) == 17854       # the island workload at 64 slots
    assert bench.bytes_per_world_step(17, 16, 3, 128) == 31486      # and at its 128


def test_traffic_from_profiles():
    for workload in ("config4", "config5"):
        t = bench.traffic_from_profiles("k_step", workload)
        text = (ROOT / "profiles" / f"k_step_{workload}_traffic.txt").read_text()
        assert t is not None and f"bytes_per_launch: {int(t)}" in text
    assert bench.traffic_from_profiles("k_step", "no_such_workload") is None


def test_toi_tail_statistics():
    """Histograms and the idle share of event waves from a State's per-world event counts (no further steps)."""
    s, m, st, cfg = b2.scenes.make_config(4, 32)
    ev = np.zeros(32, np.int32)
    ev[[0, 9, 10, 31]] = [3, 1, 2, 1]  # waves of 8 worlds: maxima 3, 2, 0, 1
    st = st._replace(toi=st.toi._replace(events=ev))
    out = bench.toi_tail(st, None, None, None, 0, 0)
    assert out["events_hist_last_step"] == [28, 2, 1, 1]
    assert out["wave_max_hist_last_step"] == [1, 1, 1, 1]
    # busy waves hold 3 + 3 + 1 = 7 world-events in 8 x (3 + 2 + 1) = 48 slots
    assert abs(out["wave_idle_frac"] - (1 - 7 / 48)) < 1e-12
    assert "steps" not in out


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=ROOT, timeout=300)
    assert r.returncode != 0 and "one GPU" in (r.stdout + r.stderr)
