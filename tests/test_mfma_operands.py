"""Every MFMA kernel of the library, compiled for gfx950 with the package's
flags, keeps its MFMA operand tuples intact (tests/mfma_operands.py): no
register of a loaded operand is overwritten before the MFMA reads it. The
checker itself is pinned on small listings with and without such an
overwrite."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT
import mfma_operands

CSRC = os.path.join(ROOT, "yue2-mlx_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
         "-target-feature", "-Xclang", "-packed-fp32-ops", "--offload-device-only", "-S"]
SOURCES = ["attention.hip", "prefill.hip", "nar_attention.hip", "gemm.hip", "gemv_mfma.hip"]

CLEAN = """_Zk:
	global_load_dwordx4 v[2:5], v[10:11], off
	ds_read_b128 v[6:9], v12
	v_cndmask_b32_e32 v3, v3, v20, vcc
	v_mul_f32_e32 v21, v3, v22
	v_or_b32_e32 v30, v40, v41
	v_or_b32_e32 v31, v40, v42
	v_or_b32_e32 v32, v40, v43
	v_or_b32_e32 v33, v40, v44
	v_mfma_f32_16x16x32_bf16 a[0:3], v[2:5], v[30:33], a[0:3]
	v_mfma_f32_16x16x32_bf16 a[4:7], v[6:9], v[30:33], a[4:7]
.Lfunc_end0:
"""


def test_checker_flags_an_overwritten_operand_register():
    count, bad = mfma_operands.check_function(CLEAN.splitlines()[1:])
    assert count == 2 and not bad
    # v4 of the loaded tile reused as a temporary before the MFMA
    clobbered = CLEAN.replace("v_mul_f32_e32 v21, v3, v22", "v_mul_f32_e32 v4, v3, v22")
    count, bad = mfma_operands.check_function(clobbered.splitlines()[1:])
    assert count == 2 and len(bad) == 1 and "v[2:5]" in bad[0][0]
    # a tile assembled from two different loads
    mixed = CLEAN.replace("ds_read_b128 v[6:9], v12", "ds_read_b128 v[6:9], v12\n\tds_read_b32 v7, v13")
    _, bad = mfma_operands.check_function(mixed.splitlines()[1:])
    assert len(bad) == 1 and "v[6:9]" in bad[0][0]


@pytest.mark.skipif(not os.path.exists(HIPCC) and not shutil.which("hipcc"), reason="no hipcc")
@pytest.mark.parametrize("source", SOURCES)
def test_mfma_operand_tuples_intact(source, tmp_path):
    out = tmp_path / (source + ".s")
    run = subprocess.run([HIPCC, *FLAGS, os.path.join(CSRC, source), "-o", str(out)],
                         capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stderr[-2000:]
    total, problems = 0, []
    for name, lines in mfma_operands.functions(out.read_text()):
        count, bad = mfma_operands.check_function(lines)
        total += count
        problems += [(name, b) for b in bad]
    assert total > 0, "no MFMA found"
    assert not problems, problems[:3]
