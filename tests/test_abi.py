"""CPU checks of the drop-in boundary: the built libraries load and
libqasr_hip.so exports exactly the entry points include/qasr_hip.h declares
(no compute calls — there is no GPU in the CPU suite)."""
import ctypes
import os
import re

from conftest import ROOT


def declared():
    src = open(os.path.join(ROOT, "include", "qasr_hip.h")).read()
    return sorted(set(re.findall(r"\b(qasr_hip_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from qwenasr_amd import _lib
    L = ctypes.CDLL(_lib.LIB_PATH)
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding covers every declared entry point
    assert set(names) <= set(_lib.declared_symbols()), set(names) - set(_lib.declared_symbols())


def test_no_cpu_fallback_in_product():
    """The product package never imports the oracle."""
    pkg = os.path.join(ROOT, "qwenasr_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h", ".c")):
                txt = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in txt.replace("Oracle", ""), f


def test_synth_and_oracle_load():
    from oracle import oracle
    from qwenasr_amd import synth
    oracle.lib()
    a = synth.normal_f32(1000, 1, "x")
    b = synth.normal_f32(1000, 1, "x")
    assert (a == b).all() and abs(float(a.std()) - 1.0) < 0.1
    c = synth.normal_bf16((4, 1 << 21), 2, "big")
    synth._synth().qs_set_threads(1)
    d = synth.normal_bf16((4, 1 << 21), 2, "big")
    synth._synth().qs_set_threads(8)
    assert (c == d).all()                      # block streams: thread count does not matter


def build_c_smoke(out_dir):
    """gcc, C99 pedantic with warnings as errors, against include/qasr_hip.h
    and the two built libraries: the header is plain C and the library links
    from C (the c_api.rs / jni_api.rs / Dart FFI pass-through callers)."""
    import subprocess
    lib_dir = os.path.join(ROOT, "qwenasr_amd")
    exe = os.path.join(str(out_dir), "c_abi_smoke")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "c_abi_smoke.c"),
                    "-L", lib_dir, "-lqasr_hip", "-lqasr_synth", "-Wl,-rpath," + lib_dir, "-o", exe],
                   check=True, capture_output=True, text=True)
    return exe


def test_c_smoke_builds_and_header_is_c_and_cxx(tmp_path):
    import subprocess
    assert os.access(build_c_smoke(tmp_path), os.X_OK)
    hdr = os.path.join(ROOT, "include", "qasr_hip.h")
    for cmd in (["gcc", "-std=c99", "-pedantic", "-Werror", "-Wall", "-x", "c", "-fsyntax-only", hdr],
                ["g++", "-std=c++17", "-pedantic", "-Werror", "-Wall", "-x", "c++", "-fsyntax-only", hdr]):
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_integration_ffi_block_is_current():
    """The Rust FFI module embedded in the integration notes is the
    generator's output for the current header: one declaration per entry
    point, nothing elided."""
    import re
    from qwenasr_amd import ffi_rust
    header = open(os.path.join(ROOT, "include", "qasr_hip.h")).read()
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"<!-- ffi:begin -->\n```rust\n(.*?)```\n<!-- ffi:end -->", doc, re.S)
    assert m, "INTEGRATION.md has no generated FFI block"
    assert m.group(1) == ffi_rust.render(header)
    n_decl = len(re.findall(r"^\s*pub fn qasr_hip_\w+\(", m.group(1), re.M))
    n_header = len(set(re.findall(r"\b(qasr_hip_\w+)\s*\(", ffi_rust.strip_comments(header))))
    assert n_decl == n_header


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N > 1 exits with status 2 and says why, before touching a GPU."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
