"""CPU-side checks of the C ABI: libvtq.so loads and exports exactly what
include/vtq.h declares; host logic that needs no GPU behaves."""
import ctypes
import os
import re
import subprocess

import pytest

import vtq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vtq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vtq_[a-z0-9_]+)\s*\(", text)))


def test_library_built_and_loads():
    assert os.path.exists(vtq.LIB_PATH), "run __graft_entry__.build()"
    lib = vtq.load_library()
    # 0.2.0: vtqrt_run takes the trailing digest_v1 argument; 0.3.0 adds
    # vtqrt_set_prompt_mode (include/vtq.h)
    assert lib.vtq_version().decode().startswith("vtq 0.3.")


def test_every_declared_symbol_is_exported():
    decl = declared_functions()
    assert len(decl) >= 10
    out = subprocess.run(["nm", "-D", "--defined-only", vtq.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\sT\s+(vtq_\w+)", out.stdout))
    missing = [f for f in decl if f not in exported]
    assert not missing, missing
    extra = sorted(f for f in exported if f not in decl)
    assert not extra, f"exported but not declared in include/vtq.h: {extra}"
    assert sorted(vtq.EXPORTED) == decl


def test_header_constants_match_python_mirror():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (VTQ_\w+) (\d+)", text))
    assert int(consts["VTQ_TYPE_Q4_K"]) == vtq.Q4_K and int(consts["VTQ_TYPE_Q6_K"]) == vtq.Q6_K
    assert int(consts["VTQ_TYPE_Q8_0"]) == vtq.Q8_0 and int(consts["VTQ_TYPE_Q5_0"]) == vtq.Q5_0
    assert int(consts["VTQ_TYPE_Q4_0"]) == vtq.Q4_0 and int(consts["VTQ_TYPE_F32"]) == vtq.F32
    assert int(consts["VTQ_E_INTERNAL"]) == vtq.Internal.code
    assert int(consts["VTQ_E_GPU"]) == vtq.GpuError.code
    assert int(consts["VTQ_E_NOT_IMPLEMENTED"]) == vtq.NotImplementedDtype.code


def test_null_context_is_rejected_without_touching_the_gpu():
    lib = vtq.load_library()
    assert lib.vtq_linear(None, vtq.Q4_K, 0, None, 0, None, 0, None, 0, 0, 0, 0) == vtq.E_INVALID_ARGUMENT
    assert lib.vtq_linear_device(None, vtq.Q4_K, 0, None, None, 0, None, 0, 0, 0, None) == vtq.E_INVALID_ARGUMENT
    assert lib.vtq_create(0, None) == vtq.E_INVALID_ARGUMENT
    assert b"null" in lib.vtq_last_error(None)


def test_no_device_maps_to_gpu_error():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(vtq.GpuError):
        vtq.Context(0)


def test_product_has_no_oracle_or_cpu_fallback():
    # libvtq must not link or load the oracle, and the package must not import it.
    for lib in (vtq.LIB_PATH, os.path.join(vtq.LIB_DIR, "libvtq_runtime.so")):
        out = subprocess.run(["ldd", lib], capture_output=True, text=True)
        assert "oracle" not in out.stdout
    pkg = os.path.dirname(vtq.__file__)
    for root, _, files in os.walk(os.path.dirname(pkg)):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".c", ".cpp")):
                src = open(os.path.join(root, f)).read()
                assert "import oracle" not in src and "vtq_oracle" not in src, f


def test_runtime_library_exports_its_header():
    from vtq import runtime

    header = os.path.join(ROOT, "include", "vtq_runtime.h")
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    decl = sorted(set(re.findall(r"\b(vtqrt_[a-z0-9_]+)\s*\(", text)))
    path = os.path.join(vtq.LIB_DIR, "libvtq_runtime.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True)
    exported = sorted(set(re.findall(r"\sT\s+(vtqrt_\w+)", out.stdout)))
    assert decl == exported
    lib = runtime.lib()
    assert lib.vtqrt_run(None, 0, b"m", None, None, 1, 1, None, None, None, None) == vtq.E_INVALID_ARGUMENT
    assert b"null" in lib.vtqrt_last_error(None)
    # the prompt mode needs a model and one of the two documented values
    assert lib.vtqrt_set_prompt_mode(None, runtime.PROMPT_BATCHED) == vtq.E_INVALID_ARGUMENT


def test_runtime_blake3_matches_oracle_on_cpu():
    import numpy as np

    import oracle
    from vtq import runtime

    data = (np.arange(70000) % 251).astype(np.uint8)
    for n in (0, 1, 1024, 1025, 70000):
        assert runtime.blake3(data[:n]).hex() == oracle.blake3(data[:n])
