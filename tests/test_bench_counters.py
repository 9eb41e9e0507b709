"""bench.py's counter plumbing on the CPU: kernel-name shortening, the
per-launch MFMA figures, the FETCH/WRITE copy calibration and the report's
handling of absent rocprofv3 runs.  The counter values here are synthetic;
the formulas are the ones documented in the report header."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("q38m_bench_under_test",
                                                  os.path.join(ROOT, "bench.py"))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_short_kernel_names(bench):
    assert bench._short_kernel(
        "void q38m::(anonymous namespace)::dense_gemm_kernel<2u, 2u, "
        "(q38m::(anonymous namespace)::DenseOut)0>(unsigned short const*, unsigned int)"
    ) == "dense_gemm_kernel<2u, 2u, DenseOut=0>"
    assert bench._short_kernel(
        "q38m::(anonymous namespace)::gate_up_w4g32_f16_kernel<2048u, 512u, false>"
        "(HIP_vector_type<unsigned int, 4u> const*)"
    ) == "gate_up_w4g32_f16_kernel<2048u, 512u, false>"
    assert bench._short_kernel("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"


def test_mfma_metrics(bench):
    agent = {"simds": 1024, "xccs": 8, "cus": 256}
    # two launches of 100 us; 8 XCCs x 200,000 busy cycles each
    cs = {
        "GRBM_GUI_ACTIVE": [1.6e6, 1.6e6],
        "SQ_INSTS_MFMA": [1.0e6, 1.0e6],
        "SQ_INSTS_VALU": [9.0e6, 9.0e6],  # includes the MFMAs
        "SQ_VALU_MFMA_BUSY_CYCLES": [1.6e7, 1.6e7],
        "SQ_INSTS_VALU_MFMA_MOPS_I8": [0.0, 0.0],
        "SQ_INSTS_VALU_MFMA_MOPS_F16": [1.0e9, 1.0e9],
        "_duration_us": [100.0, 100.0],
    }
    m = bench.mfma_metrics(cs, agent)
    assert m["launches"] == 2
    assert m["gui_active_cycles_per_xcc"] == 200000
    assert m["mfma_busy_frac"] == pytest.approx(1.6e7 / (2e5 * 1024), abs=1e-4)
    assert m["valu_insts_per_mfma"] == pytest.approx(8.0)
    assert m["valu_issue_share_est"] == pytest.approx(8e6 * 4 / (2e5 * 1024), abs=1e-4)
    ops = 1.0e9 * 512
    assert m["mfma_type"] == "fp16"
    assert m["int8_tops_counter"] == pytest.approx(ops / 100e-6 / 1e12, rel=1e-3)
    assert m["int8_peak_frac_counter"] == pytest.approx(ops / 100e-6 / 1e12 / 5000.0, abs=1e-4)
    assert m["fp16_peak_frac_counter"] == pytest.approx(ops / 100e-6 / 1e12 / 2500.0, abs=1e-4)


def test_copy_calibration(bench):
    # the copy kernel of 256 MiB reads back half its bytes in FETCH_SIZE (KiB)
    mib = 256
    agg = {("__amd_rocclr_copyBuffer", 512): {"FETCH_SIZE": [mib * 1024 / 2] * 5},
           ("__amd_rocclr_copyBuffer", 64): {"FETCH_SIZE": [3.0]},
           ("gate_up_w4_kernel", 1): {"FETCH_SIZE": [1.0]}}
    assert bench._copy_scale(agg, "FETCH_SIZE", mib) == pytest.approx(2.0)
    assert bench._copy_scale({}, "FETCH_SIZE", mib) is None


def test_pick_prefers_most_launches_or_largest_grid(bench):
    agg = {("gate_up_w4_kernel<2048u>", 100): {"_duration_us": [1.0] * 3},
           ("gate_up_w4_kernel<2048u>", 900): {"_duration_us": [1.0]},
           ("down_w8_kernel<2048u>", 5): {"_duration_us": [1.0]}}
    assert bench.pick(agg, "gate_up_w4_kernel")[0] == 100
    assert bench.pick(agg, "gate_up_w4_kernel", largest_grid=True)[0] == 900
    assert bench.pick(agg, "combine_kernel") is None


def test_report_without_rocprofv3(bench, monkeypatch):
    monkeypatch.setattr(bench.shutil, "which", lambda name: None)
    assert bench.pmc_run(bench.PMC_MFMA, "slab") is None
    assert bench.counters_summary() is None
    report = bench.pmc_report("slab")
    assert "python3 bench.py --pmc-report slab" in report
    assert "not available" in report


def test_counter_sets_fit_one_pass(bench):
    # rocprofv3 does not split counters over passes: at most 8 SQ counters
    # and 2 GRBM counters per run
    for counters in (bench.PMC_MFMA, bench.PMC_WAITS):
        names = counters.split()
        assert sum(n.startswith("SQ_") for n in names) <= 8
        assert sum(n.startswith("GRBM_") for n in names) <= 2
        assert len(set(names)) == len(names)


def test_contract_ceilings(bench):
    """The chain alone (4 VALU per fp16 MFMA) caps the W4 g32 path at half
    the int8 peak; 8 VALU per MFMA halves that again."""
    c = bench.contract_ceilings({"valu_insts_per_mfma": 8.0, "int8_peak_frac_counter": 0.15})
    assert c["chain_only_int8_frac"] == 0.5
    assert c["valu_issue_int8_frac"] == 0.25
    assert c["mfma_type"] == "fp16"
    assert bench.contract_ceilings({"valu_insts_per_mfma": 2.0,
                                    "int8_peak_frac_counter": 0.1})["valu_issue_int8_frac"] == 0.5


def test_ordered_line_ends_with_both_halves_of_the_metric(bench):
    result = {"metric": "m", "value": 1.0, "unit": "tok/s", "config": {}, "extra": 1,
              "roofline": {"frac": 0.7},
              "cpu_baseline": {"value": 2.0, "per_config": {"config1": {}}},
              "decode": {"us_per_layer": 10.0, "GBps": 2000.0, "hbm_frac": 0.25,
                         "floor": {"layer_us": 6.0, "two_launch_us": 3.2}}}
    line = bench.ordered_line(result)
    keys = list(line)
    assert keys[:4] == ["metric", "value", "unit", "config"]
    assert keys[-3:] == ["roofline", "cpu_baseline", "decode"]
    assert "per_config" not in line["cpu_baseline"]
    assert line["cpu_baseline_per_config"] == {"config1": {}}
    assert line["decode_detail"]["us_per_layer"] == 10.0
    assert line["decode"]["floor_over_measured"] == 0.6
