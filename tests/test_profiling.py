"""CPU: the rocprofv3 counter summary that scales FETCH_SIZE / WRITE_SIZE by the calibration copy."""

from __future__ import annotations

import csv

import pytest

from kv_skill_v2_amd import profiling

COLS = ["Kernel_Name", "Counter_Name", "Counter_Value"]


def _csv(path, counter, rows):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=COLS)
        w.writeheader()
        for name, val in rows:
            w.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": val})
    return str(path)


def test_traffic_scales_by_the_blit_copy(tmp_path):
    gib = 1 << 30
    conv = "void at::native::vectorized_elementwise_kernel<4, at::native::float16_copy_kernel_cuda>"
    fetch = _csv(tmp_path / "f.csv", "FETCH_SIZE",
                 [(conv, 163855.0), ("xenc::decode_read_kernel", 1000.0), ("xenc::decode_read_kernel", 1200.0),
                  ("__amd_rocclr_copyBuffer", 640.0)] + [("__amd_rocclr_copyBuffer", 524288.0)] * 3)
    write = _csv(tmp_path / "w.csv", "WRITE_SIZE",
                 [(conv, 163840.0), ("xenc::decode_read_kernel", 10.0), ("xenc::decode_read_kernel", 30.0)]
                 + [("__amd_rocclr_copyBuffer", 1048576.0)] * 3)
    res = profiling.traffic(fetch, write, "decode_read_kernel", gib)
    assert res["fetch_scale"] == pytest.approx(2.0)
    assert res["write_scale"] == pytest.approx(1.0)
    assert res["fetch_bytes"] == pytest.approx(1100.0 * 1024 * 2)
    assert res["write_bytes"] == pytest.approx(20.0 * 1024)
    assert res["dispatches"] == 2


def test_traffic_refuses_a_run_without_the_calibration_copy(tmp_path):
    conv = "void at::native::vectorized_elementwise_kernel<4, at::native::float16_copy_kernel_cuda>"
    rows = [(conv, 163855.0), ("xenc::write_back_kernel", 207419.0), ("__amd_rocclr_copyBuffer", 640.0)] * 3
    fetch = _csv(tmp_path / "f.csv", "FETCH_SIZE", rows)
    write = _csv(tmp_path / "w.csv", "WRITE_SIZE", rows)
    with pytest.raises(SystemExit):
        profiling.traffic(fetch, write, "write_back_kernel", 1 << 30)
