"""The C ABI: include/gptq2d.h compiles as C and C++, libgptq2d.so exports every symbol it declares, and
every gptq2d_* symbol the library exports is declared (loaded with ctypes and read with nm; no compute
call, so this runs without a GPU)."""

import ctypes
import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gptq2d.h"
LIB = ROOT / "gptq-2d_amd" / "libgptq2d.so"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set()
    for name in re.findall(r"\b(gptq2d_\w+)\s*\(", text):
        if "##SUF" in text and name.endswith("_"):
            continue
        names.add(name)
    for stem in re.findall(r"\b(gptq2d_\w+)_##SUF\s*\(", text):
        names.update({f"{stem}_f32", f"{stem}_f64"})
    return sorted(names)


def test_header_compiles():
    for compiler, lang in (("gcc", "c"), ("g++", "c++")):
        if shutil.which(compiler) is None:
            pytest.skip(f"{compiler} missing")
        res = subprocess.run([compiler, "-x", lang, "-fsyntax-only", "-Wall", "-Werror", str(HEADER)],
                             capture_output=True, text=True)
        assert res.returncode == 0, res.stderr


def test_library_exports_declared_symbols():
    if not LIB.exists():
        pytest.skip("libgptq2d.so is not built (run __graft_entry__.build())")
    names = declared_symbols()
    assert len(names) > 30
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def exported_symbols():
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm missing")
    res = subprocess.run([nm, "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True)
    return sorted({line.split()[-1] for line in res.stdout.splitlines()
                   if line.split() and line.split()[-1].startswith("gptq2d_")})


def test_every_export_is_declared():
    if not LIB.exists():
        pytest.skip("libgptq2d.so is not built (run __graft_entry__.build())")
    exported = exported_symbols()
    assert len(exported) > 30
    undeclared = sorted(set(exported) - set(declared_symbols()))
    assert not undeclared, undeclared
