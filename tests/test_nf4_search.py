"""The kernels' O(log 16) nearest-code search equals the reference's linear
scan (quant.rs:263-278) for every float target in [-1, 1] and the special
values -- checked exhaustively on the host, where the same header compiles.
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_search_exhaustive(tmp_path):
    exe = tmp_path / "nf4_search_check"
    obj = tmp_path / "oracle.o"
    flags = ["-O2", "-ffp-contract=off", "-fno-fast-math"]
    subprocess.run(["gcc", *flags, "-c", os.path.join(ROOT, "oracle", "qlora_oracle.c"),
                    "-o", str(obj)], check=True)
    subprocess.run(["g++", *flags, "-fopenmp", "-std=c++17",
                    "-I", os.path.join(ROOT, "vkqlora.rs_amd", "csrc"),
                    "-I", os.path.join(ROOT, "oracle"),
                    os.path.join(ROOT, "tests", "nf4_search_check.cpp"), str(obj),
                    "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "mismatches=0" in r.stdout
