"""Checks on the gfx950 code that hipcc generates around hand-written asm.

The Q8_0 LDS kernels (q8_lds_kernel<NWIN> in canon_gemv.hip) set m0, the LDS
base of `buffer_load ... lds`, inside inline asm.  m0 is a reserved register:
the compiler does not save it around an asm statement, so the kernels are
only correct while no compiler-generated instruction in them uses m0.  This
test compiles the file for gfx950 with the library's flags and checks every
instantiation.  CPU only (hipcc cross-compiles without a GPU).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "vitni-tensor_amd", "csrc", "canon_gemv.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# the device flags of vitni-tensor_amd/Makefile
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _functions(asm_text):
    """{symbol: [instruction lines]} for every function in an assembly listing."""
    out, name, body = {}, None, []
    for line in asm_text.split("\n"):
        m = re.match(r"^([_A-Za-z][\w.$]*):", line)
        if m and not line.startswith(".L"):
            name, body = m.group(1), []
            out[name] = body
        elif line.startswith(".Lfunc_end"):
            name = None
        elif name is not None:
            body.append(line.strip())
    return out


@pytest.fixture(scope="module")
def canon_asm(tmp_path_factory):
    if not (os.path.exists(HIPCC) or shutil.which("hipcc")):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "canon_gemv.s"
    subprocess.run([HIPCC if os.path.exists(HIPCC) else "hipcc", *FLAGS, "--cuda-device-only", "-S", "-o", str(out), SRC],
                   check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=600)
    return _functions(out.read_text())


def test_q8_lds_kernels_use_m0_only_in_their_lds_loads(canon_asm):
    kernels = {k: v for k, v in canon_asm.items() if "q8_lds_kernel" in k}
    assert len(kernels) == 16, sorted(kernels)  # NWIN = 1..16
    for name, body in kernels.items():
        code = [l for l in body if l and not l.startswith((";", "."))]
        n_loads = 0
        for i, line in enumerate(code):
            if not re.search(r"\bm0\b", line):
                continue
            # the asm's own pair: s_mov_b32 m0, sN ; s_nop 0 ; buffer_load_dword[x4] ... lds
            assert re.match(r"s_mov_b32 m0, s\d+$", line), (name, line)
            nxt = code[i + 1:i + 3]
            assert nxt and nxt[0] == "s_nop 0", (name, nxt)
            assert re.match(r"buffer_load_dword(x4)? v\d+, s\[\d+:\d+\], 0 offen lds$", nxt[1]), (name, nxt)
            n_loads += 1
        assert n_loads > 0, name



def _scratch_sizes(src):
    """{kernel symbol: private segment bytes per lane} of one source file."""
    out = subprocess.run([HIPCC if os.path.exists(HIPCC) else "hipcc", *FLAGS, "--cuda-device-only", "-S", "-o", "-",
                          src], check=True, stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, timeout=600).stdout
    sizes, cur = {}, None
    for line in out.decode().split("\n"):
        m = re.match(r"^([_A-Za-z][\w.$]*):", line)
        if m and not line.startswith(".L"):
            cur = m.group(1)
        m = re.match(r"^; ScratchSize: (\d+)", line.strip())
        if m and cur:
            sizes[cur] = int(m.group(1))
    return sizes


@pytest.mark.parametrize("name", ["kquant_gemv.hip", "canon_gemv.hip"])
def test_gemv_kernels_do_not_spill(name):
    # a value spilled to scratch memory is reloaded through the memory
    # hierarchy; in the GEMVs such a reload sat on the critical path
    if not (os.path.exists(HIPCC) or shutil.which("hipcc")):
        pytest.skip("hipcc not available")
    sizes = _scratch_sizes(os.path.join(ROOT, "vitni-tensor_amd", "csrc", name))
    kernels = {k: v for k, v in sizes.items() if "kernel" in k}
    assert kernels, name
    spilled = {k: v for k, v in kernels.items() if v}
    assert not spilled, spilled
