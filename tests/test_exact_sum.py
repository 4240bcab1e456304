"""The integer-state emulation of a sequential fp32 sum (pz_exact.h, used by
every GPU normaliser and CDF) reproduces plain fp32 addition bit for bit.

Pinned by the mathematics it restates: the expected value of every step is
the host's own IEEE fp32 addition (SSE, round to nearest even) of the same
two operands, over long softmax-like and sorted sequences, constructed
half-grid ties, subnormals and an edge-value grid."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "native", "exact_sum_check.cpp")
INC = os.path.join(ROOT, "project-zero_amd", "csrc")


def test_integer_state_matches_fp32_addition(tmp_path):
    exe = tmp_path / "exact_sum_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I", INC, SRC, "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout[-2000:]
    assert "0 mismatches" in out.stdout
