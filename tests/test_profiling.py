"""The rocprofv3 summary helpers (CPU only, synthetic counter files)."""

import csv

from redpanda_amd import profiling


def _write(path, rows):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(["Kernel_Name", "Counter_Name", "Counter_Value"], r)))


def test_short_name():
    assert profiling.short_name("void rp::scan_bwd_kernel<8, 5, rp::GateKind<4, 1, 4> >"
                                "(rp::ScanParams, rp::BwdIO)") == "scan_bwd_kernel"
    assert profiling.short_name("rp::bwd_reduce_bc(float const*, float*)") == "bwd_reduce_bc"
    # the step tile kernel's two beta forms stay apart
    full = "void rp::step_tile_kernel<4, 5, rp::GateKind<4, 1, 4>, true, false, false, false>(rp::StepParams)"
    rank1 = "void rp::step_tile_kernel<4, 5, rp::GateKind<4, 1, 4>, true, true, true, false>(rp::StepParams)"
    shared = "void rp::step_tile_kernel<4, 5, rp::GateKind<4, 1, 4>, true, false, false, true>(rp::StepParams)"
    assert profiling.short_name(full) == "step_tile_kernel"
    assert profiling.short_name(rank1) == "step_tile_kernel[rank1]"
    assert profiling.short_name(shared) == "step_tile_kernel[shared]"


def test_traffic_scales_by_the_calibration_dispatch(tmp_path):
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    neg = "void at::native::vectorized_elementwise_kernel<neg_kernel>(int)"
    _write(f, [(neg, "FETCH_SIZE", 512.0), ("void rp::k<1>(int)", "FETCH_SIZE", 100.0),
               ("void rp::k<1>(int)", "FETCH_SIZE", 300.0)])
    _write(w, [(neg, "WRITE_SIZE", 1024.0), ("void rp::k<1>(int)", "WRITE_SIZE", 50.0)])
    t = profiling.traffic(str(f), str(w), calib_bytes=1024 * 1024)
    assert t["calibration"]["fetch_scale"] == 2.0 and t["calibration"]["write_scale"] == 1.0
    k = t["kernels"]["k"]
    assert k["fetch_bytes"] == 200.0 * 1024 * 2.0  # mean of the two dispatches, scaled
    assert k["write_bytes"] == 50.0 * 1024


def test_valu_means_per_kernel(tmp_path):
    p = tmp_path / "v.csv"
    _write(p, [("void rp::scan_fwd_kernel<8>(int)", "SQ_INSTS_VALU", 10.0),
               ("void rp::scan_fwd_kernel<8>(int)", "SQ_INSTS_VALU", 30.0),
               ("void rp::scan_fwd_kernel<8>(int)", "SQ_WAVES", 4.0),
               ("neg_kernel", "SQ_INSTS_VALU", 99.0)])
    v = profiling.valu(str(p))["kernels"]
    assert v == {"scan_fwd_kernel": {"SQ_INSTS_VALU": 20.0, "SQ_WAVES": 4.0}}
