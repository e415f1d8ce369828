"""Shader clock of the MI355X as the amdgpu driver reports it.

MI355X's published peaks are quoted at 2400 MHz; under a sustained MFMA
workload the clock settles lower, so a rate is compared with the peak at the
clock it ran at.  bench.py reports it per workload and the cost calibration
(frisk_amd/calibrate.py) converts kernel times to cycles with it."""
from __future__ import annotations

import glob
import threading
import time


def _sclk_paths():
    return sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))


def read_sclk_mhz():
    """Current shader clock from the amdgpu driver's DPM table (the level
    marked '*'), or None where the file is not readable."""
    for path in _sclk_paths():
        try:
            for line in open(path).read().splitlines():
                if line.rstrip().endswith("*"):
                    return int(line.split(":")[1].strip().lower().split("mhz")[0])
        except (OSError, ValueError, IndexError):
            continue
    return None


def sustained_clock(torch, fn, seconds=0.4):
    """Median shader clock (MHz) sampled every 20 ms while fn runs back to
    back for `seconds` (the clock a sustained workload sees; MI355X's
    published peaks are quoted at 2400 MHz)."""
    samples, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            v = read_sclk_mhz()
            if v is not None:
                samples.append(v)
            time.sleep(0.02)

    th = threading.Thread(target=sample, daemon=True)
    th.start()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    stop.set()
    th.join()
    if not samples:
        return None
    samples.sort()
    return samples[len(samples) // 2]
