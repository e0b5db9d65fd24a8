"""Sanity of the MI355X machine file and of the probe that writes it.

The CPU test reads the committed `machines/mi355x.gpu`; the GPU test runs
`kvforge_amd/bin/bw_probe --quick` and checks the same relations on what it
measures: HBM latency clearly above the MALL-resident latency (a chase that
stays in the 256 MiB memory-side cache would make them equal), bandwidths
below the published 8 TB/s, a one-CU rate far below the device's, a
128-byte transaction.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _parse(text):
    out = {}
    for line in text.splitlines():
        line = line.split("#", 1)[0].strip()
        if "=" in line:
            k, v = (x.strip() for x in line.split("=", 1))
            out[k] = v
    return out


def _check(m):
    f = lambda k: float(m[k])  # noqa: E731
    assert int(m["wave_size"]) == 64 and int(m["sms"]) == 256
    assert f("lat_ns") > 1.3 * f("lat_mall_ns"), (m["lat_ns"], m["lat_mall_ns"])
    assert 250 <= f("lat_ns") <= 2000
    assert 4000 <= f("bw_peak_gbs") <= 8000
    assert f("bw_sm_gbs") * 20 < f("bw_peak_gbs")
    assert f("bw_copy_gbs") <= 8000 and f("bw_l2_gbs") > f("bw_peak_gbs")
    assert int(m["sector_bytes"]) in (64, 128)
    assert f("kernel_floor_us") > 0 and "round_trip_us" not in m


def test_committed_machine_file():
    with open(os.path.join(ROOT, "machines", "mi355x.gpu")) as fh:
        m = _parse(fh.read())
    _check(m)
    assert m["resources"] == "resources_gfx950.csv"


@pytest.mark.gpu
def test_probe_measures_hbm_not_the_mall(tmp_path):
    exe = os.path.join(ROOT, "kvforge_amd", "bin", "bw_probe")
    assert os.access(exe, os.X_OK), "build kvforge_amd first"
    out = tmp_path / "m.gpu"
    print("  running bw_probe --quick", flush=True)
    r = subprocess.run([exe, "--quick", "--out", str(out), "--resources", "resources_gfx950.csv"],
                       capture_output=True, text=True, timeout=150)
    print(r.stdout[-1500:], flush=True)
    assert r.returncode == 0, r.stderr[-2000:]
    _check(_parse(out.read_text()))
