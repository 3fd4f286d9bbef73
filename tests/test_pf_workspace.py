"""The prefill workspace bookkeeping behind the drop-in attn_prefill (qwengine_amd/csrc/pf_workspace.hpp), on the
CPU: growing a reservation never frees a buffer a captured graph may still hold, release frees each buffer exactly
once, and a failed allocation leaves the reservation unchanged (tests/pf_ws_check.cpp, built with g++)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_pf_workspace_bookkeeping(tmp_path):
    exe = str(tmp_path / "pf_ws_check")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    "-I", os.path.join(ROOT, "qwengine_amd", "csrc"), os.path.join(HERE, "pf_ws_check.cpp"), "-o", exe],
                   check=True)
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "pf_workspace ok" in r.stdout
