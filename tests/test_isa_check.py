"""The build-time scan of k_mx_mfma's inline-assembly loads
(stream-pt_amd/csrc/isa_check.py) on small synthetic kernels: a clean
schedule passes; a copy, a spill or an overwrite of a load register between
the issue and the wait fails."""
import importlib.util
import os

import pytest

_PATH = os.path.join(os.path.dirname(__file__), "..", "stream-pt_amd", "csrc", "isa_check.py")
_spec = importlib.util.spec_from_file_location("isa_check", _PATH)
isa_check = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(isa_check)

NAME = "_ZN3spt9k_mx_mfmaILi0EEEvNS_10MxMfmaArgsEPKiS3_S3_S3_S3_"


def kernel(inside_loop="", before_wait=""):
    issue = """\ts_nop 4
\tbuffer_load_dwordx4 v[40:43], v1, s[8:11], s12 offen
\tbuffer_load_dwordx4 v[44:47], v1, s[8:11], s12 offen offset:1024
\tbuffer_load_dwordx4 v[48:51], v1, s[8:11], s12 offen offset:2048
\tbuffer_load_dwordx4 v[52:55], v1, s[8:11], s12 offen offset:3072
"""
    return f"""{NAME}:
\tv_mov_b32_e32 v1, 0
{issue}.LBB0_1:                                ; =>This Loop Header: Depth=1
{before_wait}\ts_waitcnt vmcnt(0) ; spt tile wait
\tds_write_b128 v2, v[40:43]
\tds_write_b128 v2, v[44:47] offset:1024
\tds_write_b128 v2, v[48:51] offset:2048
\tds_write_b128 v2, v[52:55] offset:3072
\tv_add_u32_e32 v40, 1, v40
{issue}\tv_mfma_scale_f32_16x16x128_f8f6f4 v[0:3], v[4:7], v[8:15], 0, v16, v17
{inside_loop}\ts_cbranch_scc1 .LBB0_1
\ts_endpgm
.Lfunc_end0:
"""


def run(text, tmp_path):
    p = tmp_path / "k.s"
    p.write_text(text)
    return isa_check.main(str(p))


def test_clean_schedule_passes(tmp_path):
    # v40 is reused after the stores and before the next issue: allowed
    assert run(kernel(), tmp_path) == 0


@pytest.mark.parametrize("bad", ["\tv_mov_b32_e32 v60, v45\n",
                                 "\tscratch_store_dword off, v52, off\n",
                                 "\tv_mov_b32_e32 v41, 0\n"])
def test_touching_a_load_register_in_flight_fails(tmp_path, bad):
    assert run(kernel(inside_loop=bad), tmp_path) == 1
    assert run(kernel(before_wait=bad), tmp_path) == 1


def kernel_two_waits(bad_at=None):
    """Two tile waits (a prologue one, then one in the loop) and issues in
    the prologue and in the loop, as in a kernel that stores part of its
    tiles before its main loop."""
    issue = """\ts_nop 4
\tbuffer_load_dwordx4 v[40:43], v1, s[8:11], s12 offen
\tbuffer_load_dwordx4 v[44:47], v1, s[8:11], s12 offen offset:1024
\tbuffer_load_dwordx4 v[48:51], v1, s[8:11], s12 offen offset:2048
\tbuffer_load_dwordx4 v[52:55], v1, s[8:11], s12 offen offset:3072
"""
    wait = "\ts_waitcnt vmcnt(0) ; spt tile wait\n"
    stores = """\tds_write_b128 v2, v[40:43]
\tds_write_b128 v2, v[44:47] offset:1024
\tds_write_b128 v2, v[48:51] offset:2048
\tds_write_b128 v2, v[52:55] offset:3072
"""
    parts = {k: (bad_at == k and "\tv_mov_b32_e32 v60, v45\n" or "") for k in ("prologue", "loop_top", "loop_end")}
    return f"""{NAME}:
\tv_mov_b32_e32 v1, 0
{issue}{parts['prologue']}{wait}{stores}{issue}.LBB0_1:                                ; =>This Loop Header: Depth=1
{parts['loop_top']}{wait}{stores}\tv_add_u32_e32 v40, 1, v40
{issue}\tv_mfma_scale_f32_16x16x128_f8f6f4 v[0:3], v[4:7], v[8:15], 0, v16, v17
{parts['loop_end']}\ts_cbranch_scc1 .LBB0_1
\ts_endpgm
.Lfunc_end0:
"""


def test_two_waits_clean_passes(tmp_path):
    assert run(kernel_two_waits(), tmp_path) == 0


@pytest.mark.parametrize("where", ["prologue", "loop_top", "loop_end"])
def test_two_waits_touch_in_flight_fails(tmp_path, where):
    assert run(kernel_two_waits(where), tmp_path) == 1
