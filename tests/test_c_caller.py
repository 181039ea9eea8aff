# SPDX-License-Identifier: Apache-2.0
"""A plain C99 program (tests/c/k3_caller.c) compiled against include/k3.h and linked to
libk3amd.so makes the reference kernel benchmark's two calls (benchmarks/bench_kernels.c:
102-145 of the reference) with that benchmark's inputs. On the CPU: it builds from the
header alone and every symbol it needs is exported. On the GPU: its outputs, on host and on
registered (resident) weights, are within 1e-4 ||ref||inf of the oracle's, whose outputs
hash to the reference's published FNV values (tests/test_oracle.py)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import max_err_rel_inf

HERE = os.path.dirname(os.path.abspath(__file__))
CDIR = os.path.join(HERE, "c")
BIN = os.path.join(CDIR, "k3_caller")
LIB = os.path.join(os.path.dirname(HERE), "kimi-k3-in-c_amd", "libk3amd.so")


def _syms(path, flag):
    out = subprocess.run(["nm", "-D", flag, path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_c_caller_builds_against_the_header(tmp_path):
    exe = tmp_path / "k3_caller"
    subprocess.run(["gcc", "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror",
                    "-I" + os.path.join(os.path.dirname(HERE), "include"),
                    os.path.join(CDIR, "k3_caller.c"), "-o", str(exe),
                    "-L" + os.path.dirname(LIB), "-lk3amd"], check=True)
    need = {s for s in _syms(str(exe), "--undefined-only") if s.startswith("k3")}
    assert {"k3_matmul_bf16", "k3_matmul_mxfp4", "k3_dev_register", "k3_dev_unregister"} <= need
    assert need <= _syms(LIB, "--defined-only")


def test_integration_snippet_compiles(tmp_path):
    """The resident-weights example of the integration guide compiles against the header
    with the exported signatures."""
    subprocess.run(["gcc", "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-c",
                    "-I" + os.path.join(os.path.dirname(HERE), "include"),
                    os.path.join(CDIR, "k3_resident_snippet.c"), "-o", str(tmp_path / "s.o")],
                   check=True)
    src = open(os.path.join(CDIR, "k3_resident_snippet.c")).read()
    guide = open(os.path.join(os.path.dirname(HERE), "INTEGRATION.md")).read()
    for line in ("k3_dev_register(w->gate, (size_t)c->n_experts * c->hidden * sizeof(float));",
                 "k3_moe(out, x, w, c, T, idx, wt, scratch);"):
        assert line in src and line in guide


@pytest.mark.gpu
def test_c_caller_outputs(gpu, orc, tmp_path):
    assert os.path.exists(BIN), "tests/c/k3_caller is built by __graft_entry__.build()"
    out = tmp_path / "y.bin"
    r = subprocess.run([BIN, str(out)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stderr
    y = np.fromfile(out, np.float32)
    assert y.size == 2 * 12288 + 2 * 3072
    W = orc.fill_bf16(7168 * 12288, 12345).reshape(12288, 7168)
    x = orc.fill_f(7168, 999)
    want = orc.matmul_bf16(x, W)
    assert orc.fnv1a(want) == 0x83C8504A4CB3FAC6
    assert max_err_rel_inf(y[:12288], want) <= 1e-4
    assert max_err_rel_inf(y[12288:24576], want) <= 1e-4
    pk = orc.fill_b(3072 * 1792, 777)
    sc = np.full(3072 * 112, 127, np.uint8)
    xm = orc.fill_f(3584, 4242)
    wm = orc.matmul_mxfp4(xm, pk, sc, 3584, 3072)
    assert orc.fnv1a(wm) == 0xA231061237B5579D
    assert max_err_rel_inf(y[24576:27648], wm) <= 1e-4
    assert max_err_rel_inf(y[27648:], wm) <= 1e-4
    assert "k3_expert_drops = 0" in r.stdout
