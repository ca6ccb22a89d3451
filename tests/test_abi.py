"""The C-ABI library builds, loads and exports exactly what include/ferrum_hip.h
declares (CPU only: nothing here launches a kernel)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ferrum_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_python_exports():
    import ferrum_hip

    assert declared() == sorted(ferrum_hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    import ferrum_hip

    out = subprocess.run(["nm", "-D", "--defined-only", ferrum_hip.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared() if s not in syms]
    assert not missing, missing


def test_library_loads_and_binds():
    import ferrum_hip

    L = ferrum_hip.lib()
    for s in declared():
        assert getattr(L, s) is not None


def test_header_compiles_as_c():
    src = '#include "ferrum_hip.h"\nint main(void){ fh_sampling_params p = {0.8f, 40, 0.95f, 1.1f}; return (int)p.top_k - 40; }\n'
    exe = "/tmp/fh_header_check"
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), "-x", "c", "-",
                        "-o", exe], input=src, text=True, capture_output=True)
    assert r.returncode == 0, r.stderr
    assert subprocess.run([exe]).returncode == 0


def test_rng_matches_the_oracle(orc):
    import ferrum_hip

    for seed in (0, 1, 42, 2**63 + 5):
        a, b = ferrum_hip.Rng(seed), orc.Rng(seed)
        for _ in range(50):
            assert a.next_u64() == b.next_u64()
        assert a.next_f32() == b.next_f32()


def test_sampling_params_layout_matches_the_header():
    import ctypes
    import ferrum_hip

    assert ctypes.sizeof(ferrum_hip.SamplingParams) == 16
    p = ferrum_hip.SamplingParams(0.8, 40, 0.95, 1.1)
    assert (p.top_k, round(p.temperature, 6)) == (40, 0.8)


def test_numerics_constants_match_the_header():
    """The Python and Rust numerics codes are the header's enum."""
    import ferrum_hip

    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    enum = dict((k, int(v)) for k, v in re.findall(r"\bFH_(W8A32_EXACT|W8A8_FAST|W8A32|W8A8)\s*=\s*(\d+)", text))
    assert enum == {"W8A32": ferrum_hip.W8A32, "W8A8": ferrum_hip.W8A8, "W8A32_EXACT": ferrum_hip.W8A32_EXACT,
                    "W8A8_FAST": ferrum_hip.W8A8_FAST}
    rust = open(os.path.join(ROOT, "ferrum-cpu_amd", "rust", "ferrum_hip", "src", "lib.rs")).read()
    for name, code in enum.items():
        assert re.search(rf"pub const FH_{name}: c_int = {code};", rust), name
