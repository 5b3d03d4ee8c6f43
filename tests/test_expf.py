"""The device routing's expf (fm_expf_ref, flash-moe_amd/csrc/fm_expf.h) is
bit-equal to the libm expf that the oracle and the compiled reference call
(cpu_softmax / cpu_sigmoid, cpu_kernels.h:258-277): the header is compiled for
the host and compared over EVERY non-NaN float input (4.28e9 values, both
signs; ~10 s on 8 threads)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_expf_ref_matches_libm_exhaustively(tmp_path):
    exe = str(tmp_path / "expf_check")
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-o", exe,
                    os.path.join(HERE, "expf_check", "expf_check.cpp"), "-lm"], check=True)
    r = subprocess.run([exe, "1"], capture_output=True, text=True, timeout=600)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    assert r.stdout.strip() == "checked 4278190082 mismatches 0"
