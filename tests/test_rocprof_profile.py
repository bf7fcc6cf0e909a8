"""rocprofv3 evidence behind ``--profile-candidate --rocprof``.

CPU tests: the CSV parser and region split on hand-made rocprofv3 output, the
pass command lines, and the CLI's parent side end to end against a stand-in
``rocprofv3`` that writes such output (no GPU, no profiler).
"""

import csv
import os
import stat
import sys
import textwrap
from pathlib import Path

import pytest

from tiktoktechjam2026track3_amd import profiling, runner

TRACE_FIELDS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id",
                "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
COUNTER_FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
                  "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size",
                  "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value",
                  "Start_Timestamp", "End_Timestamp"]

COPY = profiling.COPY_KERNEL
MARK = "void at::cuda::(anonymous namespace)::spin_kernel(long)"
GEMM = "void enc::(anonymous namespace)::gemm_big_kernel<256, 256, 32, 4, 4, 1>(unsigned short const*)"
ATTN = "void enc::(anonymous namespace)::attn_fwd_kernel<64, 4, false, 0, true, true, 0, 4>(float)"

# (dispatch id, kernel, duration ns): a calibration copy, one warmup call, then
# the profiled region of case A (two calls), then case B's warmup and region.
DISPATCHES = [
    (1, COPY, 40000), (2, GEMM, 999), (3, ATTN, 999),
    (4, MARK, 10), (5, GEMM, 1000), (6, ATTN, 3000), (7, GEMM, 1400), (8, ATTN, 3400), (9, MARK, 10),
    (10, GEMM, 999),
    (11, MARK, 10), (12, ATTN, 500), (13, MARK, 10),
]


def write_trace(directory: Path):
    directory.mkdir(parents=True)
    with open(directory / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=TRACE_FIELDS, quoting=csv.QUOTE_NONNUMERIC)
        w.writeheader()
        t = 1000
        for did, name, dur in DISPATCHES:
            w.writerow({"Kind": "KERNEL_DISPATCH", "Agent_Id": "Agent 1", "Queue_Id": 1, "Stream_Id": 0,
                        "Thread_Id": 1, "Dispatch_Id": did, "Kernel_Id": 1, "Kernel_Name": name,
                        "Correlation_Id": did, "Start_Timestamp": t, "End_Timestamp": t + dur})
            t += dur + 100


def write_counters(directory: Path, values):
    """values: {counter: {kernel: value per dispatch}}"""
    directory.mkdir(parents=True)
    with open(directory / "run_counter_collection.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=COUNTER_FIELDS)
        w.writeheader()
        for did, name, _ in DISPATCHES:
            for counter, per_kernel in values.items():
                value = per_kernel.get(name, 1.0)
                if callable(value):
                    value = value(did)
                w.writerow({"Correlation_Id": did, "Dispatch_Id": did, "Agent_Id": "Agent 1", "Queue_Id": 1,
                            "Process_Id": 1, "Thread_Id": 1, "Grid_Size": 1, "Kernel_Id": 1, "Kernel_Name": name,
                            "Workgroup_Size": 256, "LDS_Block_Size": 0, "Scratch_Size": 0, "VGPR_Count": 8,
                            "Accum_VGPR_Count": 0, "SGPR_Count": 16, "Counter_Name": counter,
                            "Counter_Value": value, "Start_Timestamp": 0, "End_Timestamp": 0})


def write_all(root: Path, copy_mib: int = 256):
    write_trace(root / "trace")
    copy_units = copy_mib * 1024.0  # 1 KiB per unit for the copy
    # FETCH_SIZE in 2-KiB units (scale 2048 bytes/unit), WRITE_SIZE in 1-KiB units
    write_counters(root / "fetch", {"FETCH_SIZE": {COPY: copy_units / 2, GEMM: lambda d: 100.0 if d < 7 else 300.0,
                                                    ATTN: 50.0}})
    write_counters(root / "write", {"WRITE_SIZE": {COPY: copy_units, GEMM: 64.0, ATTN: 10.0}})
    # busy cycles over (GUI_ACTIVE / 8 XCDs x 1024 SIMDs): GEMM 0.5, ATTN 0.25
    write_counters(root / "mfma", {"SQ_VALU_MFMA_BUSY_CYCLES": {GEMM: 0.5 * 1024 * 1000, ATTN: 0.25 * 1024 * 1000},
                                   "GRBM_GUI_ACTIVE": {GEMM: 8000.0, ATTN: 8000.0}})


def test_regions_keep_only_the_dispatches_between_marker_pairs(tmp_path):
    write_trace(tmp_path / "trace")
    regions = profiling.profiled_regions(profiling.read_dispatches(str(tmp_path / "trace")))
    assert [[d.id for d in r] for r in regions] == [[5, 6, 7, 8], [12]]
    assert [d.duration_ns for d in regions[0]] == [1000, 3000, 1400, 3400]


def test_unterminated_region_is_an_error(tmp_path):
    write_trace(tmp_path / "trace")
    dispatches = profiling.read_dispatches(str(tmp_path / "trace"))[:-1]
    with pytest.raises(ValueError, match="no end marker"):
        profiling.profiled_regions(dispatches)


def test_summary_per_kernel(tmp_path):
    write_all(tmp_path)
    dirs = {name: str(tmp_path / name) for name, _ in profiling.ROCPROF_PASSES}
    cases = profiling.summarize_rocprof(dirs, {"trace": "cmd"}, 2)
    assert len(cases) == 2
    a = cases[0]
    assert a["calibration"]["fetch_bytes_per_unit"] == pytest.approx(2048.0)
    assert a["calibration"]["write_bytes_per_unit"] == pytest.approx(1024.0)
    assert a["kernel_time_ms"] == pytest.approx((1000 + 3000 + 1400 + 3400) / 1e6)
    by = {k["kernel"]: k for k in a["kernels"]}
    assert [k["kernel"] for k in a["kernels"]] == [ATTN, GEMM]  # by total time
    g, t = by[GEMM], by[ATTN]
    assert g["calls"] == 2 and g["avg_us"] == pytest.approx(1.2)
    assert g["share"] == pytest.approx(2400 / 8800)
    # dispatch 5 reads 100 units and dispatch 7 reads 300 (warmup dispatch 2 is left out)
    assert g["fetched_bytes_per_call"] == pytest.approx(200 * 2048.0)
    assert g["written_bytes_per_call"] == pytest.approx(64 * 1024.0)
    assert g["hbm_gbps"] == pytest.approx((200 * 2048.0 + 64 * 1024.0) / 1200.0)
    assert g["mfma_busy"] == pytest.approx(0.5)
    assert t["mfma_busy"] == pytest.approx(0.25)
    assert g["name"].startswith("gemm_big_kernel<256, 256, 32, 4, 4, 1>")
    b = cases[1]
    assert [k["calls"] for k in b["kernels"]] == [1]


def test_region_count_must_match_the_cases(tmp_path):
    write_all(tmp_path)
    dirs = {name: str(tmp_path / name) for name, _ in profiling.ROCPROF_PASSES}
    with pytest.raises(ValueError, match="expected 3"):
        profiling.summarize_rocprof(dirs, {}, 3)


def test_pass_commands_profile_the_interpreter_directly():
    cmds = profiling.rocprof_commands("/out", ["--encoder-configs", "c2", "--profile-candidate", "--rocprof"])
    assert [name for name, _ in cmds] == ["trace", "fetch", "write", "mfma"]
    for name, cmd in cmds:
        program = cmd[cmd.index("--") + 1:]
        # the profiled program is the interpreter binary itself, no launcher hop
        assert os.path.basename(program[0]).startswith("python")
        assert not os.path.islink(program[0])
        assert program[1:3] == ["-m", "tiktoktechjam2026track3_amd.runner"]
        assert program[-1] == "--rocprof-child"
        flags = cmd[1:cmd.index("--output-format")]
        # a kernel trace alone, or one counter set alone (within one pass's
        # hardware limits), never both in one run
        assert flags == {"trace": ["--kernel-trace"], "fetch": ["--pmc", "FETCH_SIZE"],
                         "write": ["--pmc", "WRITE_SIZE"],
                         "mfma": ["--pmc", "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]}[name]


def test_rocprof_needs_profile_candidate():
    args = runner.parse_args(["--encoder-configs", "c2", "--rocprof"])
    with pytest.raises(ValueError, match="requires --profile-candidate"):
        runner.validate_profile_focus(args)


def test_profiled_case_ids_skip_host_configs():
    args = runner.parse_args(["--encoder-configs", "c1", "c3", "--profile-candidate", "--rocprof"])
    assert runner.profiled_case_ids(args) == [3]
    args = runner.parse_args(["--official-cases", "2", "7", "--profile-candidate", "--rocprof"])
    assert runner.profiled_case_ids(args) == [2, 7]


FAKE_ROCPROF = textwrap.dedent("""\
    #!{python}
    # Stand-in for rocprofv3: writes hand-made CSV output for the pass it is
    # asked for and records its command line.
    import sys
    sys.path.insert(0, {tests!r})
    from pathlib import Path
    import test_rocprof_profile as t
    argv = sys.argv[1:]
    out = Path(argv[argv.index("-d") + 1])
    name = out.name
    root = out.parent
    root.mkdir(parents=True, exist_ok=True)
    with open(root / "commands.txt", "a") as fh:
        fh.write(" ".join(argv) + "\\n")
    scratch = root / ("_" + name)
    t.write_all(scratch)
    (scratch / name).rename(out)
    """)


def test_collect_rocprof_runs_every_pass_and_summarises(tmp_path, monkeypatch):
    bindir = tmp_path / "bin"
    bindir.mkdir()
    fake = bindir / "rocprofv3"
    fake.write_text(FAKE_ROCPROF.format(python=os.path.realpath(sys.executable),
                                        tests=str(Path(__file__).resolve().parent)))
    fake.chmod(fake.stat().st_mode | stat.S_IEXEC)
    monkeypatch.setenv("PATH", f"{bindir}{os.pathsep}{os.environ['PATH']}")
    argv = ["--encoder-configs", "c2", "c3", "--profile-candidate", "--rocprof",
            "--rocprof-dir", str(tmp_path / "prof")]
    args = runner.parse_args(argv)
    lines = []
    monkeypatch.setattr("builtins.print", lambda *a, **k: lines.append(" ".join(map(str, a))))
    result = runner.collect_rocprof(args, argv)
    assert sorted(result) == [2, 3]
    assert result[2]["kernels"][0]["calls"] == 2 and result[3]["kernels"][0]["calls"] == 1
    assert set(result[2]["passes"]) == {"trace", "fetch", "write", "mfma"}
    commands = (tmp_path / "prof" / "commands.txt").read_text().splitlines()
    assert len(commands) == 4 and all(c.endswith("--rocprof-child") for c in commands)
    assert sum("rocprofv3 pass" in line for line in lines) == 4


def test_failing_pass_reports_its_output(tmp_path, monkeypatch):
    bindir = tmp_path / "bin"
    bindir.mkdir()
    fake = bindir / "rocprofv3"
    fake.write_text(f"#!{os.path.realpath(sys.executable)}\nimport sys\nprint('no device here')\nsys.exit(3)\n")
    fake.chmod(fake.stat().st_mode | stat.S_IEXEC)
    monkeypatch.setenv("PATH", f"{bindir}{os.pathsep}{os.environ['PATH']}")
    argv = ["--encoder-configs", "c2", "--profile-candidate", "--rocprof", "--rocprof-dir", str(tmp_path / "p")]
    with pytest.raises(RuntimeError, match="status 3:\n.*no device here"):
        runner.collect_rocprof(runner.parse_args(argv), argv)


def test_short_names_keep_anonymous_namespace_kernels():
    from tiktoktechjam2026track3_amd.profiling import short_name

    assert short_name("void enc::(anonymous namespace)::gemm_big_kernel<256, 256, 32, 4, 4, 1>(unsigned short const*, int)") \
        == "gemm_big_kernel<256, 256, 32, 4, 4, 1>"
    assert short_name("void (anonymous namespace)::softmax_warp_forward<float, float, float, 7, false, false>(float*, int)") \
        == "softmax_warp_forward<float, float, float, 7, false, false>"
    assert short_name("void at::native::(anonymous namespace)::distribution_kernel<float, 4>(long, float*)") \
        == "at::native::distribution_kernel<float, 4>"
    assert short_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"
