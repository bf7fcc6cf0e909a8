"""The GEMM-vs-hipBLASLt counter summary (gemm_compare.summarize) on
synthetic rocprofv3 CSV files: the last dispatches of each kernel family are
averaged, and the clock and MFMA busy share follow from the cycle counts."""

import csv

from tiktoktechjam2026track3_amd import gemm_compare

BLAS = "Custom_Cijk_Alik_Bljk_BBS_BH_Bias_HA_S_SAV_NTD_SK3_UserArgs_MT256x256x64_MI16x16x1"
PACKED = "void enc::(anonymous namespace)::gemm_big_kernel<256, 256, 32, 4, 0, 1>(unsigned short const*, int)"
PLAIN = "void enc::(anonymous namespace)::gemm_big_kernel<256, 256, 64, 2, 0, 1>(unsigned short const*, int)"


def _trace(path, rows):
    path.mkdir()
    with open(path / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        t = 0
        for i, (name, ns) in enumerate(rows):
            w.writerow([i + 1, name, t, t + ns])
            t += ns + 1000


def _pmc(path, rows):
    path.mkdir()
    with open(path / "run_counter_collection.csv", "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, (name, counters) in enumerate(rows):
            for c, v in counters.items():
                w.writerow([i + 1, name, c, v])


def test_summary_averages_the_last_dispatches(tmp_path):
    # a probe product of the library first (ignored: only the last 3 count)
    _trace(tmp_path / "trace", [(BLAS, 999_000)] + [(BLAS, 190_000)] * 3 + [(PACKED, 220_000)] * 3
           + [(PLAIN, 230_000), (PLAIN, 230_000), (PLAIN, 233_000)])
    p1 = [(BLAS, {"GRBM_GUI_ACTIVE": 1.0, "SQ_VALU_MFMA_BUSY_CYCLES": 1.0})]
    p1 += [(BLAS, {"GRBM_GUI_ACTIVE": 8 * 380_000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 0.75 * 1024 * 380_000})] * 3
    p1 += [(PACKED, {"GRBM_GUI_ACTIVE": 8 * 440_000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * 1024 * 440_000})] * 3
    _pmc(tmp_path / "p1", p1)
    _pmc(tmp_path / "p2", [(PLAIN, {"TCP_TCC_READ_REQ_sum": 10.0}), (PLAIN, {"TCP_TCC_READ_REQ_sum": 20.0}),
                           (PLAIN, {"TCP_TCC_READ_REQ_sum": 30.0}), (PLAIN, {"TCP_TCC_READ_REQ_sum": 40.0})])
    text = gemm_compare.summarize([str(tmp_path / d) for d in ("trace", "p1", "p2")])
    rows = {line.split(" | ")[0].lstrip("| "): line for line in text.splitlines()}
    assert "| 190.0 | 220.0 | 231.0 |" in rows["time (µs, kernel trace)"]
    assert "| 3.8e+05 | 4.4e+05 | — |" in rows["shader cycles (GRBM_GUI_ACTIVE / 8 XCDs)"]
    assert "| 2.00 | 2.00 | — |" in rows["shader clock (GHz, cycles over the trace time)"]
    assert "| 75.0 | 50.0 | — |" in rows["MFMA busy (%)"]
    assert "| — | — | 30 |" in rows["TCP_TCC_READ_REQ (L1 to L2 requests)"]


def test_main_writes_the_file(tmp_path):
    _trace(tmp_path / "trace", [(BLAS, 100_000)] * 3)
    out = tmp_path / "summary.md"
    assert gemm_compare.main(["summarize", str(tmp_path / "trace"), "--out", str(out),
                              "--command", "rocprofv3 ... run 1 2 3"]) == 0
    text = out.read_text()
    assert text.startswith("# Wide GEMM against hipBLASLt")
    assert "    rocprofv3 ... run 1 2 3" in text and "| 100.0 | — | — |" in text
