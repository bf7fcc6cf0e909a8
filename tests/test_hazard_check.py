"""The build's MFMA result hazard check (hazard_check.py) on planted code.

The disassembly below is written by hand in the format llvm-objdump prints for
gfx950 code objects.  One path reads the MFMA's result two wait states after
it (the branch skips the s_nop that the fall-through path has): the check must
report exactly that read.  With the wait states in place, or with the MFMA
accumulating into the same registers (the supported back-to-back chain), it
must report nothing.
"""

from tiktoktechjam2026track3_amd import hazard_check

HEAD = "0000000000001000 <kern>:\n"


def line(addr: int, text: str, target: str = "") -> str:
    return f"\t{text:<60}// {addr:012X}: 00000000 {target}\n"


def planted(read_after_branch: bool) -> str:
    text = HEAD
    text += line(0x1000, "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]")
    text += line(0x1008, "s_cmp_eq_u32 s0, 0")
    target = "<kern+0x30>" if read_after_branch else "<kern+0x40>"
    text += line(0x100C, "s_cbranch_scc1 8", target)
    text += line(0x1010, "s_nop 7")
    text += line(0x1014, "v_mov_b32_e32 v30, 0")
    text += line(0x1030, "v_accvgpr_read_b32 v21, a3")
    text += line(0x1038, "global_store_dword v[8:9], v21, off")
    text += line(0x1040, "s_endpgm")
    return text


def test_planted_short_path_is_reported():
    report = hazard_check.check_text(planted(read_after_branch=True))
    assert report.mfmas == 1
    assert len(report.findings) == 1
    finding = report.findings[0]
    assert finding.read_addr == 0x1030 and finding.wait_states == 2
    assert "a3" in finding.read


def test_padded_paths_pass():
    # both paths reach the read only through the s_nop 7 (2 + 8 + 1 wait states)
    text = HEAD
    text += line(0x1000, "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]")
    text += line(0x1008, "s_cmp_eq_u32 s0, 0")
    text += line(0x100C, "s_cbranch_scc1 1", "<kern+0x14>")
    text += line(0x1010, "s_nop 7")
    text += line(0x1014, "s_nop 7")
    text += line(0x1018, "v_accvgpr_read_b32 v21, a3")
    text += line(0x1020, "s_endpgm")
    report = hazard_check.check_text(text)
    assert report.findings == []
    assert report.min_straight_line >= hazard_check.REQUIRED_WAIT_STATES


def test_accumulation_chain_is_not_a_read_but_an_operand_read_is():
    text = HEAD
    text += line(0x1000, "v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]")
    text += line(0x1008, "v_mfma_f32_32x32x16_bf16 v[0:15], v[24:27], v[28:31], v[0:15]")
    text += line(0x1010, "s_endpgm")
    assert hazard_check.check_text(text).findings == []
    text = HEAD
    text += line(0x1000, "v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]")
    text += line(0x1008, "v_mfma_f32_32x32x16_bf16 v[32:47], v[0:3], v[28:31], v[32:47]")
    text += line(0x1010, "s_endpgm")
    findings = hazard_check.check_text(text).findings
    assert len(findings) == 1 and findings[0].wait_states == 0


def test_packed_fp32_instructions_are_listed():
    text = HEAD
    text += line(0x1000, "v_pk_fma_f32 v[0:1], v[2:3], v[4:5], v[6:7]")
    text += line(0x1008, "v_pk_add_f16 v0, v1, v2")
    text += line(0x100C, "s_endpgm")
    report = hazard_check.check_text(text)
    assert len(report.packed_fp32) == 1 and "v_pk_fma_f32" in report.packed_fp32[0]


def test_device_pass_ignoring_the_packed_fp32_flag_fails_the_build(monkeypatch, tmp_path):
    """build_native compiles a probe kernel device-only with the build's flags
    first: the host pass's unknown-feature note is expected, the same note
    from the device pass means -packed-fp32-ops was ignored for gfx950 and
    must stop the build.  (subprocess is replaced: no compiler runs.)"""
    import subprocess

    import pytest

    from tiktoktechjam2026track3_amd import build_native

    monkeypatch.setattr(build_native, "BUILD_DIR", tmp_path)

    def fake_run(stdout_text):
        def run(cmd, **kwargs):
            assert "--cuda-device-only" in cmd
            return subprocess.CompletedProcess(cmd, 0, stdout=stdout_text)
        return run

    monkeypatch.setattr(build_native.subprocess, "run", fake_run(""))
    build_native._check_device_feature_flag("hipcc")  # silent device pass: fine
    note = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)\n"
    monkeypatch.setattr(build_native.subprocess, "run", fake_run(note))
    with pytest.raises(RuntimeError, match="ignores -packed-fp32-ops"):
        build_native._check_device_feature_flag("hipcc")
