"""CPU check of the gfx950 code built from the kernels that use the inline-asm
LDS reads of the ordered chains (CHAIN_READ8, common.hpp): compiled with the
library's own flags, no compiler-generated instruction may touch a batch's
registers before its s_waitcnt (tests/asm_chain_check.py).  A planted copy of
an in-flight register must be reported."""
import os
import shutil
import subprocess

import pytest

from asm_chain_check import check
from needle_cs_amd import build as B

SOURCES = ["needle3_step.hip"]


def device_asm(name: str, tmp_path) -> str:
    if not os.path.exists(B.HIPCC) and not shutil.which(B.HIPCC):
        pytest.skip("hipcc is not installed")
    out = tmp_path / (name + ".s")
    cmd = [B.HIPCC, *B.FLAGS, "--offload-device-only", "-S", os.path.join(B.CSRC, name), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return out.read_text()


@pytest.mark.parametrize("name", SOURCES)
def test_chain_reads_are_waited_for(name, tmp_path):
    batches, problems = check(device_asm(name, tmp_path))
    assert batches >= 3, "no inline-asm chain reads found"
    assert not problems, "\n".join(problems[:20])


def test_checker_reports_a_copy_of_an_in_flight_register():
    asm = "\n".join([
        "_Z1kv:",
        "\t;;#ASMSTART",
        "\tds_read_b128 v[4:7], v1 offset:128",
        "\tds_read_b128 v[8:11], v1 offset:128+16",
        "\t;;#ASMEND",
        "\t;;#ASMSTART",
        "\ts_waitcnt lgkmcnt(8)",
        "\t;;#ASMEND",
        "\tv_mov_b32_e32 v20, v9",
        "\t;;#ASMSTART",
        "\ts_waitcnt lgkmcnt(8)",
        "\t;;#ASMEND",
        "\ts_endpgm",
    ])
    batches, problems = check(asm)
    assert batches == 1 and len(problems) == 1 and "v_mov_b32_e32 v20, v9" in problems[0]
    # after the second wait the same copy is legal
    ok = asm.replace("\tv_mov_b32_e32 v20, v9\n", "").replace("\ts_endpgm", "\tv_mov_b32_e32 v20, v9\n\ts_endpgm")
    assert check(ok)[1] == []
